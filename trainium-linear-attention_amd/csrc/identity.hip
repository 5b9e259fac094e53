// Causal linear attention with the identity feature map, numerator only, for gfx950 (bf16):
//   y_t = sum_{u <= t} (scale q_t . k_u) v_u
// the reference's ref_identity_numerator (benchmarks/chunked_attention_benchmark.py:81-93) and
// its chunked NKI form (old/identity_linear_attn_nki_CHUNKED.py:27-59: inter-chunk Q S, masked
// intra-chunk (Q K^T) V, state S += K^T V), evaluated sequence-parallel in three passes over
// 256-token spans (4 blocks of 64 tokens, one work-group of 8 waves each):
//  1. identity_kernel<STATE = true>: the increment of every span, dS^T = V^T K over its 256 keys
//     (dv x d, fp32), written to a workspace record per span;
//  2. stats_scan_kernel: exclusive prefix of the records over the spans of a head, in place;
//  3. identity_kernel<STATE = false>: per 32-query wave in block b of a span, O^T = S^T Q^T with
//     S = the record (keys before the span) + K^T V over the span's blocks before b (an MFMA
//     product from LDS whose accumulator rows are already the A operand of S^T Q^T under a fixed
//     permutation of d, which Q^T takes on when it is loaded), split into bf16 hi + lo; plus
//     V_b^T P^T with P = mask(K_b Q^T) of the diagonal block (hi + lo); times scale at the store.
// Each pass copies the span's K and V rows global -> LDS once with buffer_load ... lds (16-byte
// chunks XOR-swizzled by row); the waves then run without synchronisation.  Operand layouts as
// in the resident sliding-window kernel: K fragments are ds_read_b128; V^T fragments, and in
// pass 1 the K^T-ordered B operand, come from the row-major rows through ds_read_b64_tr_b16 (in
// a 16-lane group, lane i receives element i % 4 of the 8-byte chunk read by lane 4 r + i / 4 as
// its element r).
#include "la_common.hpp"
#include "la_internal.hpp"
#include "la_pack.hpp"
#include "la_stage.hpp"

namespace la {

namespace {

struct IdentityParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  void* out;
  float* state;     // [BH][ns][DV * DK] fp32: span increments, then their exclusive prefixes
  int BH, N, nb, ns;   // 64-token blocks and 256-token spans per head
  float scale;
  int out_f32;
};

constexpr int kIdNW = 8;      // waves per work-group
constexpr int kIdBlocks = 4;  // 64-token blocks per work-group

// Chunk swizzles for gfx950's LDS banks (as in the resident sliding-window kernel): K rows keep
// chunk c at c ^ ((row nch / 16) mod nch), V rows of 8 chunks at c ^ (4 bit1(row)).
__device__ __forceinline__ int id_swz_k(int row, int nch) { return ((row * nch) >> 4) % nch; }
__device__ __forceinline__ int id_swz_v(int row, int nch) { return nch >= 8 ? ((row >> 1) & 1) << 2 : 0; }

template <int KS, int MT, bool STATE>
__global__ __launch_bounds__(64 * kIdNW) __attribute__((amdgpu_waves_per_eu(KS * MT <= 2 ? 6 : 2))) void identity_kernel(
    const IdentityParams p) {
  constexpr int NW = kIdNW, NBK = kIdBlocks, DK = 16 * KS, DV = 32 * MT;
  constexpr int KCH = DK / 8, VCH = DV / 8;
  constexpr int KU = BN * DK * 2 / 1024, VU = BN * DV * 2 / 1024;   // 1 KB copy units per block
  constexpr int NU = NBK * (KU + VU), UPW = (NU + NW - 1) / NW;
  constexpr int SW = DV * DK;                                      // floats per state record
  static_assert((KCH & (KCH - 1)) == 0 && (VCH & (VCH - 1)) == 0, "XOR swizzle needs power-of-two rows");
  __shared__ __attribute__((aligned(16))) uint16_t Kl[NBK][BN * DK];
  __shared__ __attribute__((aligned(16))) uint16_t Vl[NBK][BN * DV];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), h = lane >> 5, n = lane & 31;
  const int gh = (lane >> 4) & 1, gi = lane & 15;
  const int N = p.N, bh = blockIdx.y, b0 = blockIdx.x * NBK;
  const int nbk = min(NBK, p.nb - b0);
  const size_t hrow = (size_t)bh * N;
  const uint16_t* __restrict__ kg = p.k + hrow * DK;
  const uint16_t* __restrict__ vg = p.v + hrow * DV;

  // copies: unit u (wave w takes u = w, w + NW, ...) is K unit u or V unit u - NBK KU; lane l of
  // a unit fills 16-byte slot 64 part + l of its block: row slot / nch, position slot % nch,
  // holding chunk position ^ swizzle(row) of that row.  Rows >= N read as zeros.
  {
    const u32x4 rk = buffer_rsrc(kg, (u32)N * (u32)(DK * 2)), rv = buffer_rsrc(vg, (u32)N * (u32)(DV * 2));
#pragma unroll
    for (int i = 0; i < UPW; ++i) {
      const int u = w + NW * i;
      if (u >= NU) break;
      const bool isk = u < NBK * KU;
      const int uu = isk ? u : u - NBK * KU;
      const int per = isk ? KU : VU, nch = isk ? KCH : VCH, rowb = isk ? DK * 2 : DV * 2;
      const int b = uu / per, part = uu % per;
      if (b >= nbk) continue;
      const int slot = 64 * part + lane, row = slot / nch, pos = slot % nch;
      const int chunk = pos ^ (isk ? id_swz_k(row, nch) : id_swz_v(row, nch));
      const int voff = ((b0 + b) * BN + row) * rowb + 16 * chunk;
      const u32 dst = isk ? lds_addr(&Kl[b][0]) + 1024 * part : lds_addr(&Vl[b][0]) + 1024 * part;
      lds_copy16(isk ? rk : rv, dst, voff);
    }
  }

  // Transposed read of 4 rows: lane i of each 16-lane group gets column c0 + i of rows
  // r0 .. r0 + 3 (r0 = rbase + (gi >> 2) for the reading lane) of a row-major LDS block.
  typedef short v4s __attribute__((ext_vector_type(4)));
  auto tr_read = [&](const uint16_t* blk, int rows_w, int nch, bool swv, int row, int col) -> u32x2 {
    const int chunk = (col >> 3) ^ (swv ? id_swz_v(row, nch) : id_swz_k(row, nch));
    const uint16_t* src = blk + row * rows_w + 8 * chunk + (col & 7);
    const v4s r4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)src);
    return __builtin_bit_cast(u32x2, r4);
  };

  if (STATE) {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's copies landed
    __builtin_amdgcn_s_barrier();          // every wave's copies landed
    asm volatile("" ::: "memory");
    // wave w < MT * NC: dv tile w % MT, d tile w / MT, over the keys of all blocks of the span
    constexpr int NC = (DK + 31) / 32;   // 32-wide column tiles of d
    const int mt = w % MT, c = w / MT;
    if (c >= NC) return;
    {
      f32x16 acc = splat16(0.f);
      const bool colok = 32 * c + 16 * gh < DK;   // whole 16-lane groups are in or out of range
      for (int b = 0; b < nbk; ++b)
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        // keys 16 m + 8 s2 + 4 h + 0..3 for element 4 s2 + 0..3, in A (V^T) and B (K) alike
        u32 va[4], kb[4];
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const int row = 16 * m + 8 * s2 + 4 * h + (gi >> 2);
          const u32x2 vv = tr_read(&Vl[b][0], DV, VCH, true, row, 32 * mt + 16 * gh + 4 * (gi & 3));
          const u32x2 kk = tr_read(&Kl[b][0], DK, KCH, false, row, colok ? 32 * c + 16 * gh + 4 * (gi & 3) : 0);
          va[2 * s2] = vv[0];
          va[2 * s2 + 1] = vv[1];
          kb[2 * s2] = colok ? kk[0] : 0u;
          kb[2 * s2 + 1] = colok ? kk[1] : 0u;
        }
        acc = mfma32x32x16((u32x4){va[0], va[1], va[2], va[3]}, (u32x4){kb[0], kb[1], kb[2], kb[3]}, acc);
      }
      // acc: lane column d = 32 c + n, rows dv = 32 mt + c32_row(i, h)
      float* rec = p.state + ((size_t)bh * p.ns + blockIdx.x) * SW;
      if (32 * c + n < DK) {
#pragma unroll
        for (int i = 0; i < 16; ++i) rec[(32 * mt + c32_row(i, h)) * DK + 32 * c + n] = acc[i];
      }
    }
    return;
  }

  // output pass: wave w takes queries wq0 .. wq0 + 31 of block bq = w / 2
  const int bq = w >> 1;
  const int wq0 = (b0 * BN) + 32 * w;
  const bool wave_live = bq < nbk && wq0 < N;
  const bool qok = wave_live && wq0 + n < N;
  const uint16_t* __restrict__ qrow = p.q + hrow * DK + (size_t)(wq0 + n) * DK;
  // Q^T as the B operand: qf in natural order (k = 16 kk + 8 h + e, for the scores against the
  // K rows), qp in the order of the state accumulator rows (k = 16 kk + 8 (e / 4) + 4 h + e % 4)
  u32x4 qf[KS], qp[KS];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    qf[kk] = load_row8<true>(qrow, 16 * kk + 8 * h, DK, qok);
    u32x2 lo = {0u, 0u}, hi = {0u, 0u};
    if (qok) {
      lo = *reinterpret_cast<const u32x2*>(qrow + 16 * kk + 4 * h);
      hi = *reinterpret_cast<const u32x2*>(qrow + 16 * kk + 8 + 4 * h);
    }
    qp[kk] = (u32x4){lo[0], lo[1], hi[0], hi[1]};
  }
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's copies and Q rows landed
  __builtin_amdgcn_s_barrier();          // every wave's copies landed
  asm volatile("" ::: "memory");
  if (!wave_live) return;

  // O^T = S^T Q^T, one (dv tile mt, d tile c) of S at a time.  S (rows d, columns dv) starts as
  // the span's record (S^T before the span, [dv][d] fp32) in the MFMA accumulator layout (lane
  // column dv = 32 mt + n, rows d = 32 c + 8 g + 4 h + 0..3 for elements 4 g .. 4 g + 3), then
  // S += K^T V over the span's blocks before bq (MFMA A = K^T and B = V, both transposed reads
  // from the row-major blocks, keys in the same order).  For K step kk = 2 c + kk2 the lane's A
  // values are elements 8 kk2 .. 8 kk2 + 7 (rows d = 16 kk + 8 (e / 4) + 4 h + e % 4, the order
  // of qp), split into bf16 hi + lo.
  constexpr int NC = (DK + 31) / 32;
  const float* rec = p.state + ((size_t)bh * p.ns + blockIdx.x) * SW;
  f32x16 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc[mt] = splat16(0.f);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      f32x16 st;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 32 * c + 8 * g + 4 * h;
        f32x4 x = {0.f, 0.f, 0.f, 0.f};
        if (d0 < DK) x = *reinterpret_cast<const f32x4*>(rec + (32 * mt + n) * DK + d0);
#pragma unroll
        for (int e = 0; e < 4; ++e) st[4 * g + e] = x[e];
      }
      const bool colok = 32 * c + 16 * gh < DK;
      for (int jb = 0; jb < bq; ++jb)
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          u32 ka[4], vb[4];
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            const int row = 16 * m + 8 * s2 + 4 * h + (gi >> 2);
            const u32x2 kk2 = tr_read(&Kl[jb][0], DK, KCH, false, row, colok ? 32 * c + 16 * gh + 4 * (gi & 3) : 0);
            const u32x2 vv = tr_read(&Vl[jb][0], DV, VCH, true, row, 32 * mt + 16 * gh + 4 * (gi & 3));
            ka[2 * s2] = colok ? kk2[0] : 0u;
            ka[2 * s2 + 1] = colok ? kk2[1] : 0u;
            vb[2 * s2] = vv[0];
            vb[2 * s2 + 1] = vv[1];
          }
          st = mfma32x32x16((u32x4){ka[0], ka[1], ka[2], ka[3]}, (u32x4){vb[0], vb[1], vb[2], vb[3]}, st);
        }
#pragma unroll
      for (int kk2 = 0; kk2 < 2; ++kk2) {
        const int kk = 2 * c + kk2;
        if (kk >= KS) break;
        u32 hi[4], lo[4];
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          const float x0 = st[8 * kk2 + 2 * e2], x1 = st[8 * kk2 + 2 * e2 + 1];
          const u32 ph = pack_bf16x2(x0, x1);
          hi[e2] = ph;
          lo[e2] = pack_bf16x2(x0 - bf16_lo_to_f32(ph), x1 - bf16_hi_to_f32(ph));
        }
        acc[mt] = mfma32x32x16((u32x4){hi[0], hi[1], hi[2], hi[3]}, qp[kk], acc[mt]);
        acc[mt] = mfma32x32x16((u32x4){lo[0], lo[1], lo[2], lo[3]}, qp[kk], acc[mt]);
      }
    }
  }

  // diagonal block bq: keys up to the wave's last query, 32-key halves ks, causal mask
  const int query = wq0 + n;
  const int jb = bq;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int kb = (b0 + jb) * BN + 32 * ks;
    if (kb > wq0 + 31) continue;
    u32x4 kf[KS];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const int row = 32 * ks + n, c = 2 * kk + h;
      kf[kk] = *reinterpret_cast<const u32x4*>(&Kl[jb][row * DK + 8 * (c ^ id_swz_k(row, KCH))]);
    }
    f32x16 sc = splat16(0.f);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) sc = mfma32x32x16(kf[kk], qf[kk], sc);
    u32x4 phi[2], plo[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      u32 hi[4], lo[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int i0 = 8 * m + 2 * c;
        const float a = kb + c32_row(i0, h) <= query ? sc[i0] : 0.f;
        const float bb = kb + c32_row(i0 + 1, h) <= query ? sc[i0 + 1] : 0.f;
        const u32 ph = pack_bf16x2(a, bb);
        hi[c] = ph;
        lo[c] = pack_bf16x2(a - bf16_lo_to_f32(ph), bb - bf16_hi_to_f32(ph));
      }
      phi[m] = (u32x4){hi[0], hi[1], hi[2], hi[3]};
      plo[m] = (u32x4){lo[0], lo[1], lo[2], lo[3]};
    }
    // V^T fragment for keys 32 ks + 16 m + 8 (e / 4) + 4 h + e % 4 (element e), the order of the
    // score accumulator rows
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        u32 vv[4];
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const int row = 32 * ks + 16 * m + 8 * s2 + 4 * h + (gi >> 2);
          const u32x2 r2 = tr_read(&Vl[jb][0], DV, VCH, true, row, 32 * mt + 16 * gh + 4 * (gi & 3));
          vv[2 * s2] = r2[0];
          vv[2 * s2 + 1] = r2[1];
        }
        const u32x4 vf = {vv[0], vv[1], vv[2], vv[3]};
        acc[mt] = mfma32x32x16(vf, phi[m], acc[mt]);
        acc[mt] = mfma32x32x16(vf, plo[m], acc[mt]);
      }
    }
  }

  if (query < N) {
    const size_t obase = (hrow + query) * (size_t)DV;
    const float c = p.scale;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = acc[mt][4 * g + e] * c;
        store_out4<true>(p.out, p.out_f32, obase, 32 * mt + 8 * g + 4 * h, DV, y);
      }
  }
}

template <int KS, int MT>
int launch_identity_t(IdentityParams p, hipStream_t stream) {
  const dim3 grid((unsigned)p.ns, (unsigned)p.BH), block(64 * kIdNW);
  hipLaunchKernelGGL((identity_kernel<KS, MT, true>), grid, block, 0, stream, p);
  hipLaunchKernelGGL(stats_scan_kernel, dim3((unsigned)p.BH, (unsigned)(32 * MT * 16 * KS / 16)), dim3(256), 0, stream,
                     p.state, p.ns, 32 * MT * 16 * KS, 32 * MT * 16 * KS, nullptr, 0);
  hipLaunchKernelGGL((identity_kernel<KS, MT, false>), grid, block, 0, stream, p);
  return (int)hipGetLastError();
}

}  // namespace

bool identity_shape(int d, int dv) { return (d == 16 || d == 32 || d == 64) && (dv == 32 || dv == 64); }

size_t identity_workspace_bytes(int BH, int N, int d, int dv) {
  if (!identity_shape(d, dv)) return 0;
  return (size_t)BH * (((size_t)N + kIdBlocks * BN - 1) / (kIdBlocks * BN)) * (size_t)d * (size_t)dv * 4;
}

int launch_identity(const IdentityArgs& a, hipStream_t stream) {
  IdentityParams p{};
  p.q = static_cast<const uint16_t*>(a.q);
  p.k = static_cast<const uint16_t*>(a.k);
  p.v = static_cast<const uint16_t*>(a.v);
  p.out = a.out;
  p.state = static_cast<float*>(a.workspace);
  p.BH = a.BH;
  p.N = a.N;
  p.nb = (a.N + BN - 1) / BN;
  p.ns = (p.nb + kIdBlocks - 1) / kIdBlocks;
  p.scale = a.scale;
  p.out_f32 = a.out_f32 ? 1 : 0;
  const int ks = a.d / 16;
  if (a.dv == 32) {
    if (ks == 1) return launch_identity_t<1, 1>(p, stream);
    if (ks == 2) return launch_identity_t<2, 1>(p, stream);
    return launch_identity_t<4, 1>(p, stream);
  }
  if (ks == 1) return launch_identity_t<1, 2>(p, stream);
  if (ks == 2) return launch_identity_t<2, 2>(p, stream);
  return launch_identity_t<4, 2>(p, stream);
}

}  // namespace la
