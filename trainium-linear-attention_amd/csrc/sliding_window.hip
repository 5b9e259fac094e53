// Causal sliding-window softmax attention for gfx950 (bf16 and fp32 inputs).
//
// Replaces the NKI sliding-window kernel (kernels/nki_attention_sliding.py:30-132) and its
// wrapper (benchmarks/sliding_attention_benchmark.py:59-99): query t attends to keys
// t-W+1 .. t with softmax(scale * q.k) (benchmarks/sliding_attention_benchmark.py:32-56).
//
// Differences in design from the NKI kernel: no padded K/V copies and no mask tensor in HBM
// (validity comes from indices), any window size (not W <= 65), and dv independent of d.
//
// Per work-group: 4 waves x 32*QT queries.  The work-group streams the 64-key blocks that
// intersect [q0 - W + 1, q0 + BM) through LDS (double buffered, V transposed, shared with the
// parallel BASED kernel's staging).  Each wave runs an online softmax over 32-key subtiles:
// S^T = K Q^T via MFMA, running max / sum per query kept consistent across the two lane halves
// that hold the same query (one cross-half exchange per subtile), P split into bf16 hi + lo so
// that the P.V MFMAs keep ~16 mantissa bits, fp32 accumulation.
#include <float.h>

#include "la_common.hpp"
#include "la_internal.hpp"
#include "la_stage.hpp"

namespace la {

namespace {

struct SlidingParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  void* out;
  const float* addend;   // optional fp32 addend of the output (16-byte aligned), or null
  int BH, N, d, dv, window, nqb;
  float scale_log2;   // scale * log2(e)
  int out_f32;
};

template <int KS, int MT, int QT, bool VEC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(KS == 8 ? 1 : (KS == 4 && MT == 2 && QT == 1 ? 4 : 2)))) void sliding_bf16_kernel(
    const SlidingParams p) {
  constexpr int DK = 16 * KS, DV = 32 * MT, BM = 128 * QT;
  constexpr int KROW = DK + 8;
  using Stager = BlockStager<KS, MT, VEC>;

  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][BN * KROW];
  __shared__ __attribute__((aligned(16))) uint16_t VTs[2][DV * VROW];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), h = lane >> 5, n = lane & 31;
  const int N = p.N, d = p.d, dv = p.dv, W = p.window;

  int bh, qb;
  map_causal_block(blockIdx.x, p.BH, p.nqb, bh, qb);
  const int q0 = qb * BM;
  const int jlo = max(0, q0 - W + 1) / BN;
  const int jhi = min((N - 1) / BN, (q0 + BM - 1) / BN);
  const size_t hrow = (size_t)bh * N;
  const uint16_t* __restrict__ qg = p.q + hrow * d;
  const uint16_t* __restrict__ kg = p.k + hrow * d;
  const uint16_t* __restrict__ vg = p.v + hrow * dv;

  const int wq0 = q0 + 32 * QT * w;
  const bool wave_live = wq0 < N;
  const int wlo = wq0 - W + 1;             // lowest key any query of this wave can see

  u32x4 qf[QT][KS];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int query = wq0 + 32 * qt + n;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
      qf[qt][kk] = load_row8<VEC>(qg + (size_t)query * d, 16 * kk + 8 * h, d, query < N);
  }

  f32x16 acc[QT][MT];
  float mrun[QT], lrun[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[qt][mt] = splat16(0.f);
    mrun[qt] = -FLT_MAX;
    lrun[qt] = 0.f;
  }

  // Two key blocks of loads in flight: block j + 1 waits in registers while block j is used.
  // Look-ahead loads past jhi are issued with no rows in range (they touch no memory), so that
  // the loop body has no wave-uniform branches around loads and the wait for block j + 1 does not
  // drain the newer loads.
  Stager sa;
  sa.load(kg, vg, jlo * BN, N, d, dv, tid);
  sa.store(Ks[0], VTs[0], tid);
  __syncthreads();

  const float sl2 = p.scale_log2;
  auto block_step = [&](int j, Stager& nxt) {
    const int s = (j - jlo) & 1;
    nxt.load(kg, vg, (j + 1) * BN, j + 1 <= jhi ? N : 0, d, dv, tid);

    if (wave_live) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int kb = j * BN + 32 * ks;
        if (kb > wq0 + 32 * QT - 1 || kb + 31 < wlo) continue;
        u32x4 kf[KS];
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
          kf[kk] = *reinterpret_cast<const u32x4*>(&Ks[s][(32 * ks + n) * KROW + 16 * kk + 8 * h]);

        u32x4 phi[QT][2], plo[QT][2];
        bool act[QT];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const int qbase = wq0 + 32 * qt;
          act[qt] = (kb <= qbase + 31) && (kb + 31 >= qbase - W + 1) && (qbase < N);
          if (!act[qt]) continue;
          f32x16 sc = splat16(0.f);
#pragma unroll
          for (int kk = 0; kk < KS; ++kk) sc = mfma32x32x16(kf[kk], qf[qt][kk], sc);
          const int query = qbase + n;
          const bool inside = (kb + 31 <= qbase) && (kb >= qbase + 31 - W + 1);
          float t[16];
          float mloc = -FLT_MAX;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = kb + c32_row(i, h);
            const bool ok = inside || (key <= query && key >= query - W + 1);
            t[i] = ok ? sc[i] * sl2 : -FLT_MAX;
            mloc = fmaxf(mloc, t[i]);
          }
          mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
          const float mnew = fmaxf(mrun[qt], mloc);
          const float alpha = __builtin_amdgcn_exp2f(mrun[qt] - mnew);
          mrun[qt] = mnew;
          float l = lrun[qt] * alpha;
          float pr[16];
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float e = (t[i] == -FLT_MAX) ? 0.f : __builtin_amdgcn_exp2f(t[i] - mnew);
            pr[i] = e;
            l += e;
          }
          lrun[qt] = l;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[qt][mt][i] *= alpha;
#pragma unroll
          for (int m = 0; m < 2; ++m) {
            u32 hi[4], lo[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              const float a = pr[8 * m + 2 * c], b = pr[8 * m + 2 * c + 1];
              const u32 ph = pack_bf16x2(a, b);
              hi[c] = ph;
              lo[c] = pack_bf16x2(a - bf16_lo_to_f32(ph), b - bf16_hi_to_f32(ph));
            }
            phi[qt][m] = (u32x4){hi[0], hi[1], hi[2], hi[3]};
            plo[qt][m] = (u32x4){lo[0], lo[1], lo[2], lo[3]};
          }
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
          for (int m = 0; m < 2; ++m) {
            const uint16_t* vp = &VTs[s][(32 * mt + n) * VROW + 32 * ks + 16 * m + 4 * h];
            const u32x2 a0 = *reinterpret_cast<const u32x2*>(vp);
            const u32x2 a1 = *reinterpret_cast<const u32x2*>(vp + 8);
            const u32x4 vf = {a0[0], a0[1], a1[0], a1[1]};
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
              if (!act[qt]) continue;
              acc[qt][mt] = mfma32x32x16(vf, phi[qt][m], acc[qt][mt]);
              acc[qt][mt] = mfma32x32x16(vf, plo[qt][m], acc[qt][mt]);
            }
          }
        }
      }
    }
    if (j < jhi) nxt.store(Ks[s ^ 1], VTs[s ^ 1], tid);
    __syncthreads();
  };
  for (int j = jlo; j <= jhi; ++j) block_step(j, sa);

  if (!wave_live) return;
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const float l = lrun[qt] + __shfl_xor(lrun[qt], 32);
    const int query = wq0 + 32 * qt + n;
    if (query >= N) continue;
    const float inv = 1.0f / l;
    const size_t obase = (hrow + query) * (size_t)dv;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = acc[qt][mt][4 * g + e] * inv;
        store_out4<VEC>(p.out, p.out_f32, obase, 32 * mt + 8 * g + 4 * h, dv, y, p.addend);
      }
  }
}

// W <= 64 XB + 1, d % 16 == 0, dv % 32 == 0, q, k, v 16-byte aligned: a tile of 32 NW queries
// needs at most NW / 2 + XB 64-key blocks, so all of them are copied global -> LDS at once with buffer_load ... lds
// (K and V row-major, the 16-byte chunks of each row XOR-swizzled by the row index against bank
// conflicts) and the waves then run without further synchronisation.  K fragments (A operand of
// S^T = K Q^T) are ds_read_b128; V^T fragments (A operand of O^T = V^T P^T) come straight from
// the row-major V with ds_read_b64_tr_b16: within each 16-lane group, lane i receives element
// (i % 4) of the 8-byte chunk read by lane 4 r + i / 4 as its element r, so lane 4 r + c of the
// group reads row k0 + r, columns c0 + 4 c .. +3 and lane i ends up with column c0 + i of rows
// k0 .. k0 + 3.  Everything else (masking, online softmax, hi/lo split of P) is as in
// sliding_bf16_kernel.

// Chunk swizzles for gfx950's LDS (64 dword banks; ds_read_b128 serves lanes with equal lane >> 5
// and equal parity of lane bits 2..4 in one pass, ds_read_b64_tr_b16 32 consecutive lanes): K row
// `row` of nch 16-byte chunks keeps chunk c at c ^ ((row nch / 16) mod nch), so the fragment reads
// (lane n reads row n) put the 16 rows of a pass in distinct bank groups; a V row of 8 chunks
// keeps chunk c at c ^ (4 bit1(row)), so the transposed reads of rows r .. r + 3 (four chunks
// each) cover all 64 banks (rows of 4 chunks need no swizzle).
__device__ __forceinline__ int swz_k(int row, int nch) { return ((row * nch) >> 4) % nch; }
__device__ __forceinline__ int swz_v(int row, int nch) { return nch >= 8 ? ((row >> 1) & 1) << 2 : 0; }

template <int KS, int MT, int NW, int XB>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW == 8 ? 4 : 3))) void sliding_resident_kernel(
    const SlidingParams p) {
  constexpr int DK = 16 * KS, DV = 32 * MT, BM = 32 * NW;
  constexpr int kResBlocks = BM / BN + XB;   // key blocks a tile needs for W <= 64 XB + 1
  constexpr int KCH = DK / 8, VCH = DV / 8;                 // 16-byte chunks per K / V row
  constexpr int KU = BN * DK * 2 / 1024, VU = BN * DV * 2 / 1024;   // 1 KB copy units per block
  constexpr int NU = kResBlocks * (KU + VU), UPW = (NU + NW - 1) / NW;
  static_assert((KCH & (KCH - 1)) == 0 && (VCH & (VCH - 1)) == 0, "XOR swizzle needs power-of-two rows");
  __shared__ __attribute__((aligned(16))) uint16_t Kl[kResBlocks][BN * DK];
  __shared__ __attribute__((aligned(16))) uint16_t Vl[kResBlocks][BN * DV];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), h = lane >> 5, n = lane & 31;
  const int N = p.N, W = p.window;

  int bh, qb;
  map_causal_block(blockIdx.x, p.BH, p.nqb, bh, qb);
  const int q0 = qb * BM;
  const int jlo = max(0, q0 - W + 1) / BN;
  const int jhi = min((N - 1) / BN, (q0 + BM - 1) / BN);
  const int nbk = jhi - jlo + 1;   // <= kResBlocks for W <= 64 XB + 1
  const size_t hrow = (size_t)bh * N;
  const uint16_t* __restrict__ qg = p.q + hrow * DK;
  const uint16_t* __restrict__ kg = p.k + hrow * DK;
  const uint16_t* __restrict__ vg = p.v + hrow * DV;

  // copies: unit u (wave w takes u = w, w + NW, ...) is K unit u (blocks of KU) or V unit
  // u - kResBlocks KU;
  // lane l of a unit fills 16-byte slot 64 part + l of its block, i.e. row slot / nch, position
  // slot % nch, which holds chunk position ^ swizzle(row) of that row
  {
    const u32x4 rk = buffer_rsrc(kg, (u32)N * (u32)(DK * 2)), rv = buffer_rsrc(vg, (u32)N * (u32)(DV * 2));
#pragma unroll
    for (int i = 0; i < UPW; ++i) {
      const int u = w + NW * i;
      if (u >= NU) break;
      const bool isk = u < kResBlocks * KU;
      const int uu = isk ? u : u - kResBlocks * KU;
      const int per = isk ? KU : VU, nch = isk ? KCH : VCH, rowb = isk ? DK * 2 : DV * 2;
      const int b = uu / per, part = uu % per;
      if (b >= nbk) continue;
      const int slot = 64 * part + lane, row = slot / nch, pos = slot % nch;
      const int chunk = pos ^ (isk ? swz_k(row, nch) : swz_v(row, nch));
      const int voff = ((jlo + b) * BN + row) * rowb + 16 * chunk;
      const u32 dst = isk ? lds_addr(&Kl[b][0]) + 1024 * part : lds_addr(&Vl[b][0]) + 1024 * part;
      lds_copy16(isk ? rk : rv, dst, voff);
    }
  }

  const int wq0 = q0 + 32 * w;
  const bool wave_live = wq0 < N;
  const int wlo = wq0 - W + 1;
  u32x4 qf[KS];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) qf[kk] = load_row8<true>(qg + (size_t)(wq0 + n) * DK, 16 * kk + 8 * h, DK, wq0 + n < N);

  f32x16 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = splat16(0.f);
  float mrun = -FLT_MAX, lrun = 0.f;

  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's copies (and its Q rows) landed
  __builtin_amdgcn_s_barrier();          // every wave's copies landed
  asm volatile("" ::: "memory");

  const float sl2 = p.scale_log2;
  const int gh = (lane >> 4) & 1, gi = lane & 15;
  if (wave_live) {
    for (int b = 0; b < nbk; ++b) {
      const int j = jlo + b;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int kb = j * BN + 32 * ks;
        if (kb > wq0 + 31 || kb + 31 < wlo) continue;
        u32x4 kf[KS];
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
          const int row = 32 * ks + n, c = 2 * kk + h;
          kf[kk] = *reinterpret_cast<const u32x4*>(&Kl[b][row * DK + 8 * (c ^ swz_k(row, KCH))]);
        }
        f32x16 sc = splat16(0.f);
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) sc = mfma32x32x16(kf[kk], qf[kk], sc);
        const int query = wq0 + n;
        const bool inside = (kb + 31 <= wq0) && (kb >= wq0 + 31 - W + 1);
        float t[16];
        float mloc = -FLT_MAX;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = kb + c32_row(i, h);
          const bool ok = inside || (key <= query && key >= query - W + 1);
          t[i] = ok ? sc[i] * sl2 : -FLT_MAX;
          mloc = fmaxf(mloc, t[i]);
        }
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
        const float mnew = fmaxf(mrun, mloc);
        const float alpha = __builtin_amdgcn_exp2f(mrun - mnew);
        mrun = mnew;
        float l = lrun * alpha;
        float pr[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float e = (t[i] == -FLT_MAX) ? 0.f : __builtin_amdgcn_exp2f(t[i] - mnew);
          pr[i] = e;
          l += e;
        }
        lrun = l;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[mt][i] *= alpha;
        u32x4 phi[2], plo[2];
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          u32 hi[4], lo[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const float a = pr[8 * m + 2 * c], bb = pr[8 * m + 2 * c + 1];
            const u32 ph = pack_bf16x2(a, bb);
            hi[c] = ph;
            lo[c] = pack_bf16x2(a - bf16_lo_to_f32(ph), bb - bf16_hi_to_f32(ph));
          }
          phi[m] = (u32x4){hi[0], hi[1], hi[2], hi[3]};
          plo[m] = (u32x4){lo[0], lo[1], lo[2], lo[3]};
        }
        // V^T fragment for keys 32 ks + 16 m + 8 (e / 4) + 4 h + e % 4 (element e), the order of
        // the score accumulator rows: two transposed reads, rows 32 ks + 16 m + 8 s + 4 h + 0..3
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
          for (int m = 0; m < 2; ++m) {
            u32 vv[4];
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
              const int row = 32 * ks + 16 * m + 8 * s2 + 4 * h + (gi >> 2);
              const int col = 32 * mt + 16 * gh + 4 * (gi & 3);
              uint16_t* src = &Vl[b][row * DV + 8 * ((col >> 3) ^ swz_v(row, VCH)) + (col & 7)];
              typedef short v4s __attribute__((ext_vector_type(4)));
              const v4s r4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)src);
              const u32x2 r2 = __builtin_bit_cast(u32x2, r4);
              vv[2 * s2] = r2[0];
              vv[2 * s2 + 1] = r2[1];
            }
            const u32x4 vf = {vv[0], vv[1], vv[2], vv[3]};
            acc[mt] = mfma32x32x16(vf, phi[m], acc[mt]);
            acc[mt] = mfma32x32x16(vf, plo[m], acc[mt]);
          }
        }
      }
    }
    const float lt = lrun + __shfl_xor(lrun, 32);
    const int query = wq0 + n;
    if (query < N) {
      const float inv = 1.0f / lt;
      const size_t obase = (hrow + query) * (size_t)DV;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float y[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] = acc[mt][4 * g + e] * inv;
          store_out4<true>(p.out, p.out_f32, obase, 32 * mt + 8 * g + 4 * h, DV, y, p.addend);
        }
    }
  }
}

template <int KS, int MT, int QT>
int launch_sl(SlidingParams p, bool vec, hipStream_t stream) {
  p.nqb = (p.N + 128 * QT - 1) / (128 * QT);
  const dim3 grid((unsigned)(p.nqb * p.BH)), block(256);
  if (vec)
    hipLaunchKernelGGL((sliding_bf16_kernel<KS, MT, QT, true>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((sliding_bf16_kernel<KS, MT, QT, false>), grid, block, 0, stream, p);
  return (int)hipGetLastError();
}

template <int KS, int MT>
int launch_resident(SlidingParams p, hipStream_t stream) {
  if (p.window <= BN + 1) {
    constexpr int NW = 8;
    p.nqb = (p.N + 32 * NW - 1) / (32 * NW);
    hipLaunchKernelGGL((sliding_resident_kernel<KS, MT, NW, 1>), dim3((unsigned)(p.nqb * p.BH)), dim3(64 * NW), 0, stream, p);
  } else {
    constexpr int NW = 4;
    p.nqb = (p.N + 32 * NW - 1) / (32 * NW);
    hipLaunchKernelGGL((sliding_resident_kernel<KS, MT, NW, 2>), dim3((unsigned)(p.nqb * p.BH)), dim3(64 * NW), 0, stream, p);
  }
  return (int)hipGetLastError();
}

int dispatch_resident(const SlidingParams& p, hipStream_t stream) {
  const int ks = p.d / 16;   // 1, 2 or 4
  if (p.dv == 32) {
    if (ks == 1) return launch_resident<1, 1>(p, stream);
    if (ks == 2) return launch_resident<2, 1>(p, stream);
    return launch_resident<4, 1>(p, stream);
  }
  if (ks == 1) return launch_resident<1, 2>(p, stream);
  if (ks == 2) return launch_resident<2, 2>(p, stream);
  return launch_resident<4, 2>(p, stream);
}

template <int KS>
int dispatch_sl_mt(const SlidingParams& p, bool vec, hipStream_t stream) {
  if (p.dv <= 32) return launch_sl<KS, 1, 2>(p, vec, stream);
  if (p.dv <= 64) return launch_sl<KS, 2, 1>(p, vec, stream);
  return launch_sl<KS, 4, 1>(p, vec, stream);
}

}  // namespace

int launch_sliding_window_f32(const SlidingArgs& a, hipStream_t stream);

int launch_sliding_window(const SlidingArgs& a, hipStream_t stream) {
  if (a.in_f32) return launch_sliding_window_f32(a, stream);
  SlidingParams p{};
  p.q = static_cast<const uint16_t*>(a.q);
  p.k = static_cast<const uint16_t*>(a.k);
  p.v = static_cast<const uint16_t*>(a.v);
  p.out = a.out;
  p.addend = a.addend;
  p.BH = a.BH;
  p.N = a.N;
  p.d = a.d;
  p.dv = a.dv;
  p.window = a.window;
  p.scale_log2 = (float)((double)a.scale * 1.4426950408889634);
  p.out_f32 = a.out_f32 ? 1 : 0;
  const bool vec = (a.d % 8 == 0) && (a.dv % 4 == 0) && ((reinterpret_cast<uintptr_t>(a.q) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(a.k) & 15) == 0) && ((reinterpret_cast<uintptr_t>(a.v) & 7) == 0) &&
                   ((reinterpret_cast<uintptr_t>(a.out) & 15) == 0);
  const bool resident = a.window <= 2 * BN + 1 && (a.d == 16 || a.d == 32 || a.d == 64) && (a.dv == 32 || a.dv == 64) &&
                        ((reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.k) |
                          reinterpret_cast<uintptr_t>(a.v) | reinterpret_cast<uintptr_t>(a.out)) & 15) == 0 &&
                        (size_t)a.N * (size_t)a.d * 2 < ((size_t)1 << 31) && (size_t)a.N * (size_t)a.dv * 2 < ((size_t)1 << 31);
  if (resident) return dispatch_resident(p, stream);
  if (a.d <= 16) return dispatch_sl_mt<1>(p, vec, stream);
  if (a.d <= 32) return dispatch_sl_mt<2>(p, vec, stream);
  if (a.d <= 64) return dispatch_sl_mt<4>(p, vec, stream);
  return dispatch_sl_mt<8>(p, vec, stream);
}

}  // namespace la
