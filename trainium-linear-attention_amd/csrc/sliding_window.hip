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
        store_out4<VEC>(p.out, p.out_f32, obase, 32 * mt + 8 * g + 4 * h, dv, y);
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
  if (a.d <= 16) return dispatch_sl_mt<1>(p, vec, stream);
  if (a.d <= 32) return dispatch_sl_mt<2>(p, vec, stream);
  if (a.d <= 64) return dispatch_sl_mt<4>(p, vec, stream);
  return dispatch_sl_mt<8>(p, vec, stream);
}

}  // namespace la
