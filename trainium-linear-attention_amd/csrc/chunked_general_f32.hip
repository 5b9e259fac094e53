// Chunked BASED attention for fp32 inputs (any d <= 64, dv <= 128): the segment-state path of
// chunked_general.hip in fp32 arithmetic, on v_mfma_f32_32x32x2_f32.  The feature basis and the
// segment split are those of la_general.hpp; every product, state and sum is fp32, so no range
// scaling is needed.  The chunk recurrence is that of kernels/nki_attention_chunked.py:65-109
// with chunk = GL tokens, which gives the same function as every other chunk size.
//
// Kernel 1 (g32_state_kernel): one work-group per (head, 16 feature groups), four waves of two
// 32-feature tiles, sweeping the head's segments in 32-token chunks whose raw k and v rows are
// copied into an LDS ring (buffer_load ... lds, three chunks ahead).  Per K step (two tokens, one
// per lane half) a lane forms its feature b'_i b'_j of its token (A), reads v of its dv column
// (B) and adds the feature to its z partial.  After every segment but the last it writes the
// state so far as T[slot][feature][dv] and z[slot][feature].
// Kernel 2 (g32_out_kernel): one work-group per 128 queries (four waves of 32).  O^T += T^T
// Phi(Q)^T over the groups (T blocks of four groups copied into LDS, double-buffered; a'_i from
// an LDS copy of the queries' features, a'_j from registers), the denominator against z, then
// the quadratic form over the segment's keys up to each query; out = num / (den + eps).
#include "../../include/based_la.h"
#include "la_common.hpp"
#include "la_general.hpp"
#include "la_internal.hpp"

namespace la {
namespace {

constexpr int GC32 = 32;    // tokens per chunk of the state kernel
constexpr int GQ32 = 128;   // queries per output work-group

struct G32Params {
  const float* q;
  const float* k;
  const float* v;
  void* out;
  float* T;      // [seg-1][BH][F][DVP]
  float* Z;      // [seg-1][BH][F]
  float* Tot;    // per (part < nparts - 1, head, state work-group, thread): its part's sums
  float* den_out;   // optional (BH, N): each row's denominator without eps
  int nparts, spp;
  int BH, N, d, dv, nseg;
  float scale, eps;
  int normalize, out_f32;
};

__device__ __forceinline__ f32x16 mfma32x32x2_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void wait_vm32(int n) {
  asm volatile("" ::: "memory");
  switch (n) {
#define LA_VM(k) \
  case k: __builtin_amdgcn_s_waitcnt((((k) & 15) | (((k) >> 4) << 14)) | 0x0f70); break;
    LA_VM(0) LA_VM(1) LA_VM(2) LA_VM(3) LA_VM(4) LA_VM(5) LA_VM(6) LA_VM(7) LA_VM(8) LA_VM(9) LA_VM(10)
    LA_VM(11) LA_VM(12) LA_VM(13) LA_VM(14) LA_VM(15) LA_VM(16) LA_VM(17) LA_VM(18) LA_VM(19) LA_VM(20)
    LA_VM(21) LA_VM(22) LA_VM(23) LA_VM(24) LA_VM(25) LA_VM(26) LA_VM(27) LA_VM(28) LA_VM(29) LA_VM(30)
#undef LA_VM
    default: __builtin_amdgcn_s_waitcnt(0x0f70 | 15 | (1 << 14)); break;   // 31
  }
  asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------- kernel 1: segment states
// Sequences with few heads split the sweep into p.nparts parts of p.spp segments: a TOTAL pass
// sums every part but the last, then each part's work-group starts from the totals before it.
template <int DP, int DVT, bool TOTAL>
__global__ __launch_bounds__(256) void g32_state_kernel(const G32Params p) {
  using FT = GFeat<DP>;
  constexpr int DVP = 32 * DVT, NS = 4;
  constexpr int KU = DP / 8, VU = DVP / 8;       // 1 KB units of a chunk's k and v rows (at most)
  constexpr int SF = (KU + VU) * 256 + 64;       // floats per stage: k rows, v rows, constants
  __shared__ __attribute__((aligned(16))) float ring[NS][SF];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, n = lane & 31;
  const int nwga = FT::NWGA;
  const int units = p.BH * nwga;
  const int part = blockIdx.x / units;
  int bh, wga;
  {
    const int id = blockIdx.x - part * units;
    if ((p.BH & 7) == 0) {
      const int x = id & 7, r = id >> 3, hg = r / nwga;
      wga = r - hg * nwga;
      bh = 8 * hg + x;
    } else {
      bh = id / nwga;
      wga = id - bh * nwga;
    }
  }
  const int N = p.N, d = p.d, dv = p.dv;
  const int ku = (d * GC32 * 4 + 1023) / 1024, vu = (dv * GC32 * 4 + 1023) / 1024;
  const int voff_f = ku * 256;                   // first float of the v rows in a stage
  const int cst = (KU + VU) * 256;               // constants: 1.0 at cst, 0.0 at cst + 1

  // constants of every stage (the copies never reach them)
  for (int x = tid; x < NS * 64; x += 256) ring[x / 64][cst + (x & 63)] = (x & 63) == 0 ? 1.0f : 0.0f;

  // this lane's features: the value of dim x of token t sits at base + t * stride (stride 0 for
  // the constants: the augmented 1 at DP, zeros past d)
  int bi[2], si[2], bj[2], sj[2];
  bool tv[2];
#pragma unroll
  for (int mw = 0; mw < 2; ++mw) {
    const int tt = 8 * wga + 2 * w + mw;
    tv[mw] = tt < FT::NT;
    int i, J;
    group_ij<DP>(tv[mw] ? 2 * tt + (n >> 4) : 0, i, J);
    const int j = 16 * J + (n & 15);
    bi[mw] = i < d ? i : (i == DP ? cst : cst + 1);
    si[mw] = i < d ? d : 0;
    bj[mw] = j < d ? j : (j == DP ? cst : cst + 1);
    sj[mw] = j < d ? d : 0;
  }
  int bv[DVT], sv[DVT];
#pragma unroll
  for (int nt = 0; nt < DVT; ++nt) {
    const int col = 32 * nt + n;
    bv[nt] = col < dv ? voff_f + col : cst + 1;
    sv[nt] = col < dv ? dv : 0;
  }

  const int cps = GL / GC32;
  const int c0 = part * p.spp * cps, c1 = min((part + 1) * p.spp, p.nseg - 1) * cps;   // this part's chunks
  constexpr int PER = 2 * DVT * 16 + 2;   // a thread's sums: accumulators, then z partials
  const u32x4 rk = buffer_rsrc(p.k + (size_t)bh * N * d, (u32)((size_t)N * d * 4));
  const u32x4 rv = buffer_rsrc(p.v + (size_t)bh * N * dv, (u32)((size_t)N * dv * 4));
  const int my_units = (ku + vu) / 4 + (w < (ku + vu) % 4 ? 1 : 0);
  auto issue = [&](int c) {
    if (c >= c1) return;
    const u32 base = lds_addr(&ring[c % NS][0]);
    for (int u = w; u < ku + vu; u += 4) {
      if (u < ku)
        lds_copy16(rk, base + 1024 * u, c * (GC32 * d * 4) + 1024 * u + 16 * lane);
      else
        lds_copy16(rv, base + 4 * voff_f + 1024 * (u - ku), c * (GC32 * dv * 4) + 1024 * (u - ku) + 16 * lane);
    }
  };

  f32x16 acc[2][DVT];
  float zc[2] = {0.f, 0.f};
#pragma unroll
  for (int mw = 0; mw < 2; ++mw)
#pragma unroll
    for (int nt = 0; nt < DVT; ++nt) acc[mw][nt] = splat16(0.f);

  if (!TOTAL) {
    // the parts before this one
    for (int q = 0; q < part; ++q) {
      const float* t = p.Tot + (((size_t)q * p.BH + bh) * nwga + wga) * (256 * PER) + tid * PER;
#pragma unroll
      for (int mw = 0; mw < 2; ++mw)
#pragma unroll
        for (int nt = 0; nt < DVT; ++nt)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[mw][nt][r] += t[(mw * DVT + nt) * 16 + r];
      zc[0] += t[PER - 2];
      zc[1] += t[PER - 1];
    }
  }
  __syncthreads();
  for (int c = c0; c < c0 + NS - 1; ++c) issue(c);
  for (int gc = c0; gc < c1; ++gc) {
    wait_vm32(my_units * min(NS - 2, c1 - 1 - gc));
    __syncthreads();
    issue(gc + NS - 1);
    const float* st = &ring[gc % NS][0];
#pragma unroll 4
    for (int ks = 0; ks < GC32 / 2; ++ks) {
      const int t = 2 * ks + h;
      float vb[DVT];
#pragma unroll
      for (int nt = 0; nt < DVT; ++nt) vb[nt] = st[bv[nt] + t * sv[nt]];
#pragma unroll
      for (int mw = 0; mw < 2; ++mw) {
        const float a = st[bi[mw] + t * si[mw]] * st[bj[mw] + t * sj[mw]];
        zc[mw] += a;
#pragma unroll
        for (int nt = 0; nt < DVT; ++nt) acc[mw][nt] = mfma32x32x2_f32(a, vb[nt], acc[mw][nt]);
      }
    }

    if (!TOTAL && (gc + 1) % cps == 0) {
      const int s = gc / cps;
      const size_t slot = (size_t)s * p.BH + bh;
      constexpr int F = 16 * FT::NGP;
      float* Ts = p.T + slot * (size_t)F * DVP;
      float* Zs = p.Z + slot * (size_t)F;
#pragma unroll
      for (int mw = 0; mw < 2; ++mw) {
        const float zz = zc[mw] + __shfl_xor(zc[mw], 32);
        if (!tv[mw]) continue;
        const int tt = 8 * wga + 2 * w + mw;
#pragma unroll
        for (int nt = 0; nt < DVT; ++nt)
#pragma unroll
          for (int r = 0; r < 16; ++r) Ts[(size_t)(32 * tt + c32_row(r, h)) * DVP + 32 * nt + n] = acc[mw][nt][r];
        if (h == 0) Zs[32 * tt + n] = zz;
      }
      // the stores out before the copy waits above count this wave's copies again
      wait_vm32(0);
    }
  }
  if (TOTAL) {
    float* t = p.Tot + (((size_t)part * p.BH + bh) * nwga + wga) * (256 * PER) + tid * PER;
#pragma unroll
    for (int mw = 0; mw < 2; ++mw)
#pragma unroll
      for (int nt = 0; nt < DVT; ++nt)
#pragma unroll
        for (int r = 0; r < 16; ++r) t[(mw * DVT + nt) * 16 + r] = acc[mw][nt][r];
    t[PER - 2] = zc[0];
    t[PER - 1] = zc[1];
  }
}

// ---------------------------------------------------------------- kernel 2: outputs
template <int DP, int DVT>
__global__ __launch_bounds__(256, DVT == 4 ? 1 : 2) void g32_out_kernel(const G32Params p) {
  using FT = GFeat<DP>;
  constexpr int DB = DP / 16, DVP = 32 * DVT;
  constexpr int NR = DP + 16;                    // a'/m of the query, lane half 1 one further on
  constexpr int GB = 4;                          // groups per T block
  constexpr int TBF = GB * 16 * DVP + 256;       // floats per T stage: block, then 1 KB of z
  constexpr int NBLK = (FT::NG + GB - 1) / GB;
  constexpr int KROW = DP + 1;                   // key rows in LDS (odd stride: conflict-free)
  constexpr int KB = 32;                         // keys per block of the quadratic form
  constexpr int IBF = KB * KROW + KB * DVP;
  constexpr int BIGF = 2 * TBF > IBF ? 2 * TBF : IBF;
  __shared__ __attribute__((aligned(16))) float Aq[(DP + 1) * GQ32];
  __shared__ __attribute__((aligned(16))) float big[BIGF];
  __shared__ float wtab[FT::NGP];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, n = lane & 31;
  const int N = p.N, d = p.d, dv = p.dv;
  const int ntile = (N + GQ32 - 1) / GQ32;
  const int bh = blockIdx.x / ntile, tile = blockIdx.x - bh * ntile;
  const int t0 = tile * GQ32, s = t0 / GL, seg0 = s * GL;
  const float* __restrict__ qg = p.q + (size_t)bh * N * d;
  const float* __restrict__ kg = p.k + (size_t)bh * N * d;
  const float* __restrict__ vg = p.v + (size_t)bh * N * dv;

  // ---- the query: a' = [scale q, 1] with lane half 1 one index further on (R)
  const int tok = t0 + 32 * w + n;
  const bool tok_ok = tok < N;
  float R[NR];
#pragma unroll
  for (int x = 0; x < NR; ++x) {
    const int dim = x + h;
    float val = 0.f;
    if (dim < d) val = tok_ok ? qg[(size_t)tok * d + dim] * p.scale : 0.f;
    else if (dim == DP) val = 1.0f;
    R[x] = val;
  }
  if (h == 0) {
#pragma unroll
    for (int x = 0; x <= DP; ++x) Aq[x * GQ32 + 32 * w + n] = R[x];
  }

  f32x16 acc[DVT];
  float den = 0.f;
#pragma unroll
  for (int mt = 0; mt < DVT; ++mt) acc[mt] = splat16(0.f);

  if (s >= 1) {
    constexpr int F = 16 * FT::NGP;
    const size_t slot = (size_t)(s - 1) * p.BH + bh;
    for (int g = tid; g < FT::NGP; g += 256) wtab[g] = group_weight<DP>(g);
    const u32x4 rT = buffer_rsrc(p.T + slot * (size_t)F * DVP, (u32)((size_t)F * DVP * 4));
    const u32x4 rZ = buffer_rsrc(p.Z + slot * (size_t)F, (u32)(F * 4));
    constexpr int UT = GB * 16 * DVP / 256;     // 1 KB units of a T block
    auto issue = [&](int b) {
      const u32 base = lds_addr(&big[(b & 1) * TBF]);
      for (int u = w; u <= UT; u += 4) {
        if (u < UT)
          lds_copy16(rT, base + 1024 * u, b * (GB * 16 * DVP * 4) + 1024 * u + 16 * lane);
        else
          lds_copy16(rZ, base + GB * 16 * DVP * 4, b * (GB * 16 * 4) + 16 * lane);
      }
    };
    issue(0);
    int g = 0;
    for (int i = 0; i <= DP; ++i) {
      const float ai = Aq[i * GQ32 + 32 * w + n];
      const int js = i < DP ? (i >> 4) : 0, je = i < DP ? DB - 1 : DB;
#pragma unroll
      for (int J = 0; J <= DB; ++J) {
        if (J < js || J > je) continue;
        if (g % GB == 0) {
          asm volatile("" ::: "memory");
          __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's copies of the block
          asm volatile("" ::: "memory");
          __syncthreads();
          if (g / GB + 1 < NBLK) issue(g / GB + 1);
        }
        const float* st = &big[((g / GB) & 1) * TBF];
        const int sl = g % GB;
        const float wa = ai * wtab[g];
#pragma unroll
        for (int k2 = 0; k2 < 8; ++k2) {
          const int f = 16 * sl + 2 * k2 + h;
          const float b = wa * R[16 * J + 2 * k2];
          den = __builtin_fmaf(b, st[GB * 16 * DVP + f], den);
#pragma unroll
          for (int mt = 0; mt < DVT; ++mt) acc[mt] = mfma32x32x2_f32(st[f * DVP + 32 * mt + n], b, acc[mt]);
        }
        ++g;
      }
    }
    __syncthreads();   // every wave done with the T stages before the key blocks reuse them
  }

  // ---- keys of this segment up to the queries, 32 at a time, staged through registers
  float* Ks = big;
  float* Vs = big + KB * KROW;
  const int kend = min(t0 + GQ32, N);
  const int nblk = (kend - seg0 + KB - 1) / KB;
  const int wlast = min(t0 + 32 * w + 31, N - 1);
  constexpr int KPT = (KB * DP + 255) / 256, VPT = (KB * DVP + 255) / 256;
  float kr[KPT], vr[VPT];
  auto load_blk = [&](int kb0) {
#pragma unroll
    for (int e = 0; e < KPT; ++e) {
      const int x = tid + 256 * e, key = x / DP, dim = x % DP;
      kr[e] = (x < KB * DP && dim < d && kb0 + key < N) ? kg[(size_t)(kb0 + key) * d + dim] : 0.f;
    }
#pragma unroll
    for (int e = 0; e < VPT; ++e) {
      const int x = tid + 256 * e, key = x / DVP, col = x % DVP;
      vr[e] = (x < KB * DVP && col < dv && kb0 + key < N) ? vg[(size_t)(kb0 + key) * dv + col] : 0.f;
    }
  };
  auto store_blk = [&]() {
#pragma unroll
    for (int e = 0; e < KPT; ++e) {
      const int x = tid + 256 * e;
      if (x < KB * DP) Ks[(x / DP) * KROW + x % DP] = kr[e];
    }
#pragma unroll
    for (int e = 0; e < VPT; ++e) {
      const int x = tid + 256 * e;
      if (x < KB * DVP) Vs[x] = vr[e];
    }
  };
  load_blk(seg0);
  for (int j = 0; j < nblk; ++j) {
    const int kb = seg0 + KB * j;
    store_blk();
    __syncthreads();
    if (j + 1 < nblk) load_blk(kb + KB);
    const int tb = t0 + 32 * w;
    if (kb <= wlast && tb < N) {
      // S^T (keys x queries): A = K rows (dim 2 k2 + h), B = the query's a' (same dims)
      f32x16 sc = splat16(0.f);
#pragma unroll
      for (int k2 = 0; k2 < DP / 2; ++k2) sc = mfma32x32x2_f32(Ks[n * KROW + 2 * k2 + h], R[2 * k2], sc);
      float pv[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float x = sc[r];
        float pr = 1.0f + x + 0.5f * x * x;
        const int key = kb + c32_row(r, h);
        if (key > tb + n || key >= N) pr = 0.f;
        pv[r] = pr;
        den += pr;
      }
      // O^T += V^T P^T, two keys per step: key c32_row(r, h) for lane half h
#pragma unroll
      for (int r = 0; r < 16; ++r)
#pragma unroll
        for (int mt = 0; mt < DVT; ++mt) acc[mt] = mfma32x32x2_f32(Vs[c32_row(r, h) * DVP + 32 * mt + n], pv[r], acc[mt]);
    }
    __syncthreads();
  }

  // ---- out = num / (den + eps)
  den += __shfl_xor(den, 32);
  const float inv = p.normalize ? 1.0f / (den + p.eps) : 1.0f;
  if (tok_ok && h == 0 && p.den_out != nullptr) p.den_out[(size_t)bh * N + tok] = den;
  if (tok_ok) {
    const size_t ob = ((size_t)bh * N + tok) * dv;
#pragma unroll
    for (int mt = 0; mt < DVT; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int col = 32 * mt + c32_row(r, h);
        if (col < dv) {
          const float y = acc[mt][r] * inv;
          if (p.out_f32)
            static_cast<float*>(p.out)[ob + col] = y;
          else
            static_cast<uint16_t*>(p.out)[ob + col] = f32_to_bf16_bits(y);
        }
      }
  }
}

int dp32_of(int d) { return 16 * ((d + 15) / 16); }
int dvt32_of(int dv) { return dv <= 32 ? 1 : dv <= 64 ? 2 : 4; }

// Parts of the state sweep: when the (head, work-group) pairs fill less than half of 256 CUs,
// enough parts for two work-groups per CU (the totals pass sweeps all but the last part a second
// time, which pays only then), at least two segments per part.
void g32_parts(int BH, int nwga, int nseg, int& nparts, int& spp) {
  const int units = BH * nwga;
  const int want = units < 128 ? (512 + units - 1) / units : 1;
  nparts = max(1, min(want, (nseg - 1) / 2));
  spp = (nseg - 1 + nparts - 1) / nparts;
  nparts = (nseg - 1 + spp - 1) / spp;
}

// Workspace: T, z, then the part totals.
template <int DP>
size_t g32_bytes_dp(int BH, int nseg, int DVT, size_t* t_bytes = nullptr, size_t* z_bytes = nullptr) {
  constexpr int F = 16 * GFeat<DP>::NGP;
  const size_t nslot = (size_t)(nseg - 1) * BH;
  const auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
  int nparts, spp;
  g32_parts(BH, GFeat<DP>::NWGA, nseg, nparts, spp);
  const size_t tb = up(nslot * F * (32 * DVT) * 4), zb = up(nslot * F * 4);
  if (t_bytes) *t_bytes = tb;
  if (z_bytes) *z_bytes = zb;
  return tb + zb + up((size_t)(nparts - 1) * BH * GFeat<DP>::NWGA * 256 * (2 * DVT * 16 + 2) * 4);
}

size_t g32_bytes(int BH, int N, int d, int dv) {
  const int nseg = (N + GL - 1) / GL;
  if (nseg <= 1) return 0;
  switch (dp32_of(d)) {
    case 16: return g32_bytes_dp<16>(BH, nseg, dvt32_of(dv));
    case 32: return g32_bytes_dp<32>(BH, nseg, dvt32_of(dv));
    case 48: return g32_bytes_dp<48>(BH, nseg, dvt32_of(dv));
    default: return g32_bytes_dp<64>(BH, nseg, dvt32_of(dv));
  }
}

template <int DP, int DVT>
int launch_g32(const G32Params& p, hipStream_t stream) {
  if (p.nseg > 1) {
    const unsigned units = (unsigned)(p.BH * GFeat<DP>::NWGA);
    if (p.nparts > 1) {
      hipLaunchKernelGGL((g32_state_kernel<DP, DVT, true>), dim3(units * (unsigned)(p.nparts - 1)), dim3(256), 0,
                         stream, p);
      const int e = (int)hipGetLastError();
      if (e != 0) return e;
    }
    hipLaunchKernelGGL((g32_state_kernel<DP, DVT, false>), dim3(units * (unsigned)p.nparts), dim3(256), 0, stream, p);
    const int e = (int)hipGetLastError();
    if (e != 0) return e;
  }
  hipLaunchKernelGGL((g32_out_kernel<DP, DVT>), dim3((unsigned)(p.BH * ((p.N + GQ32 - 1) / GQ32))), dim3(256), 0,
                     stream, p);
  return (int)hipGetLastError();
}

template <int DP>
int launch_g32_dp(const G32Params& p, int DVT, hipStream_t stream) {
  switch (DVT) {
    case 1: return launch_g32<DP, 1>(p, stream);
    case 2: return launch_g32<DP, 2>(p, stream);
    default: return launch_g32<DP, 4>(p, stream);
  }
}

}  // namespace

size_t general_chunked_f32_bytes(int BH, int N, int d, int dv) {
  if (d < 1 || d > 64 || dv < 1 || dv > 128) return (size_t)-1;
  return g32_bytes(BH, N, d, dv);
}

int launch_general_chunked_f32(const ChunkedArgs& a, hipStream_t stream) {
  if (a.d < 1 || a.d > 64 || a.dv < 1 || a.dv > 128 || !a.in_f32) return LA_ERR_UNSUPPORTED_DIM;
  G32Params p{};
  p.q = static_cast<const float*>(a.q);
  p.k = static_cast<const float*>(a.k);
  p.v = static_cast<const float*>(a.v);
  p.out = a.out;
  p.den_out = a.den_out;
  p.BH = a.BH;
  p.N = a.N;
  p.d = a.d;
  p.dv = a.dv;
  p.nseg = (a.N + GL - 1) / GL;
  p.scale = a.scale;
  p.eps = a.eps;
  p.normalize = a.normalize ? 1 : 0;
  p.out_f32 = a.out_f32 ? 1 : 0;
  const int DP = dp32_of(a.d), DVT = dvt32_of(a.dv);
  if (p.nseg > 1) {
    const size_t need = g32_bytes(a.BH, a.N, a.d, a.dv);
    if (a.workspace == nullptr || a.workspace_bytes < need) return LA_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(a.workspace) & 15) return LA_ERR_BAD_ALIGNMENT;
    size_t tb = 0, zb = 0;
    int nwga = 0;
    switch (DP) {
      case 16: g32_bytes_dp<16>(a.BH, p.nseg, DVT, &tb, &zb); nwga = GFeat<16>::NWGA; break;
      case 32: g32_bytes_dp<32>(a.BH, p.nseg, DVT, &tb, &zb); nwga = GFeat<32>::NWGA; break;
      case 48: g32_bytes_dp<48>(a.BH, p.nseg, DVT, &tb, &zb); nwga = GFeat<48>::NWGA; break;
      default: g32_bytes_dp<64>(a.BH, p.nseg, DVT, &tb, &zb); nwga = GFeat<64>::NWGA; break;
    }
    g32_parts(a.BH, nwga, p.nseg, p.nparts, p.spp);
    char* ws = static_cast<char*>(a.workspace);
    p.T = reinterpret_cast<float*>(ws);
    p.Z = reinterpret_cast<float*>(ws + tb);
    p.Tot = reinterpret_cast<float*>(ws + tb + zb);
  }
  switch (DP) {
    case 16: return launch_g32_dp<16>(p, DVT, stream);
    case 32: return launch_g32_dp<32>(p, DVT, stream);
    case 48: return launch_g32_dp<48>(p, DVT, stream);
    default: return launch_g32_dp<64>(p, DVT, stream);
  }
}

}  // namespace la
