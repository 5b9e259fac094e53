// fp32-input kernels (gfx950 fp32 MFMA) for the parallel BASED path and the sliding-window
// softmax path.
//
// Same block structure as the bf16 kernels -- per query block, the causal (or windowed) key
// blocks stream through LDS, scores are computed transposed (S^T = K Q^T) so they feed the
// P.V MFMA without shuffles -- but every operand stays fp32 (v_mfma_f32_32x32x2_f32).  These
// serve fp32 callers such as the reference's own CPU-sized configuration, where bf16 rounding
// of P would not meet a 1e-4 tolerance.
//
//   BASED   (kernels/pytorch_attention.py:33-41): scores start from 1/c so b = q.k + 1/c,
//           p = 1 + (c^2/2)(b*b - 1/c^2) = 1 + s + s^2/2, causal mask, den = row sum of p.
//   SLIDING (benchmarks/sliding_attention_benchmark.py:32-56): online softmax of c*q.k over
//           keys t-W+1..t, running max/sum per query.
#include <float.h>

#include "la_common.hpp"
#include "la_internal.hpp"

namespace la {

namespace {

constexpr int BNF = 64;
constexpr int VROWF = BNF + 4;   // floats; 68 dwords -> 16-byte reads hit distinct banks

__device__ __forceinline__ f32x16 mfma32x32x2_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

struct F32Params {
  const float* q;
  const float* k;
  const float* v;
  void* out;
  float* den;
  const float* addend;   // sliding: optional fp32 addend of the output, or null
  int BH, N, d, dv, nqb, window;
  float inv_c, inv_c2, fscale, eps, scale_log2;
  int normalize, out_f32;
};

// SPLIT = 2 (BASED, small grids): two groups of four waves take the same 128 queries and every
// other key block each, with a staging double buffer per group, and add their numerators and
// row sums through LDS at the end, which halves the serial chain of key blocks of a query block.
template <int KS, int MT, bool SLIDING, int SPLIT = 1>
__global__ __launch_bounds__(256 * SPLIT) void f32_attn_kernel(const F32Params p) {
  static_assert(SPLIT == 1 || (SPLIT == 2 && !SLIDING), "key split: BASED only");
  constexpr int DK = 16 * KS, DV = 32 * MT, BM = 128, HALF = DK / 2;
  constexpr int KROW = DK + 4;
  constexpr int KCH = BNF * DK / 4;              // float4 chunks in a K block
  constexpr int KPT = (KCH + 255) / 256;
  constexpr int VGR = (DV / 4) * (BNF / 4);
  constexpr int VPT = (VGR + 255) / 256;

  __shared__ __attribute__((aligned(16))) float Ks[SPLIT][2][BNF * KROW];
  __shared__ __attribute__((aligned(16))) float VTs[SPLIT][2][DV * VROWF];

  const int tid_all = threadIdx.x, tid = SPLIT == 2 ? tid_all & 255 : tid_all;   // thread within its group
  const int grp = SPLIT == 2 ? __builtin_amdgcn_readfirstlane(tid_all >> 8) : 0;
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), h = lane >> 5, n = lane & 31;
  const int N = p.N, d = p.d, dv = p.dv, W = p.window;
  int bh, qb;
  map_causal_block(blockIdx.x, p.BH, p.nqb, bh, qb);
  const int q0 = qb * BM;
  const int jlo = SLIDING ? max(0, q0 - W + 1) / BNF : 0;
  const int jhi = min((N - 1) / BNF, (q0 + BM - 1) / BNF);
  const size_t hrow = (size_t)bh * N;
  const float* __restrict__ qg = p.q + hrow * d;
  const float* __restrict__ kg = p.k + hrow * d;
  const float* __restrict__ vg = p.v + hrow * dv;
  const int wq0 = q0 + 32 * w;
  const bool wave_live = wq0 < N;
  const int query = wq0 + n;

  // lane group h holds d-elements [HALF*h, HALF*h + HALF) of its query row
  float qf[HALF];
#pragma unroll
  for (int e = 0; e < HALF; ++e) {
    const int col = HALF * h + e;
    qf[e] = (query < N && col < d) ? qg[(size_t)query * d + col] : 0.f;
  }

  f32x16 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = splat16(0.f);
  float rsum = 0.f;        // BASED: row sum of p; SLIDING: running softmax sum
  float mrun = -FLT_MAX;   // SLIDING: running max (log2 domain)

  f32x4 kr[KPT];
  f32x4 vr[VPT][4];
  auto load = [&](int row0) {
#pragma unroll
    for (int r = 0; r < KPT; ++r) {
      const int c = tid + 256 * r;
      const int key = c / (DK / 4), col = 4 * (c % (DK / 4));
      const int row = row0 + key;
      f32x4 x = {0.f, 0.f, 0.f, 0.f};
      if (c < KCH && row < N) {
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = (col + e < d) ? kg[(size_t)row * d + col + e] : 0.f;
      }
      kr[r] = x;
    }
#pragma unroll
    for (int r = 0; r < VPT; ++r) {
      const int g = tid + 256 * r;
      const int g4 = g % (DV / 4), kg4 = g / (DV / 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = row0 + 4 * kg4 + i;
        f32x4 x = {0.f, 0.f, 0.f, 0.f};
        if (g < VGR && row < N) {
#pragma unroll
          for (int e = 0; e < 4; ++e) x[e] = (4 * g4 + e < dv) ? vg[(size_t)row * dv + 4 * g4 + e] : 0.f;
        }
        vr[r][i] = x;
      }
    }
  };
  auto store = [&](int s) {
#pragma unroll
    for (int r = 0; r < KPT; ++r) {
      const int c = tid + 256 * r;
      if (c < KCH) {
        const int key = c / (DK / 4), col = 4 * (c % (DK / 4));
        *reinterpret_cast<f32x4*>(&Ks[grp][s][key * KROW + col]) = kr[r];
      }
    }
#pragma unroll
    for (int r = 0; r < VPT; ++r) {
      const int g = tid + 256 * r;
      if (g < VGR) {
        const int g4 = g % (DV / 4), kg4 = g / (DV / 4);
#pragma unroll
        for (int c = 0; c < 4; ++c)
          *reinterpret_cast<f32x4*>(&VTs[grp][s][(4 * g4 + c) * VROWF + 4 * kg4]) =
              (f32x4){vr[r][0][c], vr[r][1][c], vr[r][2][c], vr[r][3][c]};
      }
    }
  };

  load((jlo + grp) * BNF);
  store(0);
  __syncthreads();
  const float inv_c = p.inv_c, inv_c2 = p.inv_c2, fscale = p.fscale, sl2 = p.scale_log2;

  // group grp takes key blocks jlo + grp, jlo + grp + SPLIT, ...; every thread runs the same
  // number of iterations (and barriers), a group past its last block idles in the last one
  const int niter = (jhi - jlo + SPLIT) / SPLIT;
  for (int it = 0; it < niter; ++it) {
    const int j = jlo + SPLIT * it + grp;
    const int s = it & 1;
    const bool more = SPLIT == 1 ? j < jhi : it + 1 < niter;
    if (more) load((j + SPLIT) * BNF);
    if (wave_live && (SPLIT == 1 || j <= jhi)) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int kb = j * BNF + 32 * ks;
        if (kb > wq0 + 31) continue;
        if (SLIDING && kb + 31 < wq0 - W + 1) continue;
        f32x16 b = splat16(SLIDING ? 0.f : inv_c);
        const float* kp = &Ks[grp][s][(32 * ks + n) * KROW + HALF * h];
#pragma unroll
        for (int e = 0; e < HALF; ++e) b = mfma32x32x2_f32(kp[e], qf[e], b);
        float pv[16];
        if (!SLIDING) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float u = __builtin_fmaf(b[i], b[i], -inv_c2);
            float pe = __builtin_fmaf(fscale, u, 1.0f);
            if (kb + c32_row(i, h) > query) pe = 0.f;
            pv[i] = pe;
            rsum += pe;
          }
        } else {
          float mloc = -FLT_MAX;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = kb + c32_row(i, h);
            const bool ok = key <= query && key >= query - W + 1;
            pv[i] = ok ? b[i] * sl2 : -FLT_MAX;
            mloc = fmaxf(mloc, pv[i]);
          }
          mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
          const float mnew = fmaxf(mrun, mloc);
          const float alpha = __builtin_amdgcn_exp2f(mrun - mnew);
          mrun = mnew;
          float l = rsum * alpha;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float e = (pv[i] == -FLT_MAX) ? 0.f : __builtin_amdgcn_exp2f(pv[i] - mnew);
            pv[i] = e;
            l += e;
          }
          rsum = l;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[mt][i] *= alpha;
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const f32x4 vv = *reinterpret_cast<const f32x4*>(&VTs[grp][s][(32 * mt + n) * VROWF + 32 * ks + 8 * g + 4 * h]);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[mt] = mfma32x32x2_f32(vv[e], pv[4 * g + e], acc[mt]);
          }
        }
      }
    }
    if (more) store(s ^ 1);
    __syncthreads();
  }

  if (SPLIT == 2) {
    // group 1 hands its numerators and row sums to group 0 through the (now free) stages
    float* red = &VTs[0][0][0];
    static_assert(SPLIT == 1 || 4 * (MT * 16 + 1) * 64 <= SPLIT * 2 * DV * VROWF, "reduction fits");
    if (grp == 1 && wave_live) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) red[((w * MT + mt) * 16 + i) * 64 + lane] = acc[mt][i];
      red[(4 * MT * 16 + w) * 64 + lane] = rsum;
    }
    __syncthreads();
    if (grp == 1) return;
    if (wave_live) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[mt][i] += red[((w * MT + mt) * 16 + i) * 64 + lane];
      rsum += red[(4 * MT * 16 + w) * 64 + lane];
    }
  }

  if (!wave_live) return;
  const float rs = rsum + __shfl_xor(rsum, 32);
  if (query >= N) return;
  float inv;
  if (SLIDING) {
    inv = 1.0f / rs;
  } else {
    inv = p.normalize ? 1.0f / (rs + p.eps) : 1.0f;
    if (p.den != nullptr && h == 0) p.den[hrow + query] = rs;
  }
  const size_t obase = (hrow + query) * (size_t)dv;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int col = 32 * mt + c32_row(i, h);
      if (col < dv) {
        float y = acc[mt][i] * inv;
        if (SLIDING && p.addend != nullptr) y += p.addend[obase + col];
        if (p.out_f32)
          static_cast<float*>(p.out)[obase + col] = y;
        else
          static_cast<uint16_t*>(p.out)[obase + col] = f32_to_bf16_bits(y);
      }
    }
}

template <int KS, int MT, bool SL>
int launch_f32(F32Params p, hipStream_t stream) {
  p.nqb = (p.N + 127) / 128;
  const dim3 grid((unsigned)(p.nqb * p.BH));
  if constexpr (!SL && KS == 1 && MT <= 2) {
    // fewer query blocks than CUs: split every query block's keys over two wave groups
    if ((long long)p.nqb * p.BH < device_cu_count()) {
      hipLaunchKernelGGL((f32_attn_kernel<KS, MT, SL, 2>), grid, dim3(512), 0, stream, p);
      return (int)hipGetLastError();
    }
  }
  hipLaunchKernelGGL((f32_attn_kernel<KS, MT, SL>), grid, dim3(256), 0, stream, p);
  return (int)hipGetLastError();
}

template <int KS, bool SL>
int dispatch_f32_mt(const F32Params& p, hipStream_t stream) {
  if (p.dv <= 32) return launch_f32<KS, 1, SL>(p, stream);
  if (p.dv <= 64) return launch_f32<KS, 2, SL>(p, stream);
  return launch_f32<KS, 4, SL>(p, stream);
}

template <bool SL>
int dispatch_f32(const F32Params& p, hipStream_t stream) {
  if (p.d <= 16) return dispatch_f32_mt<1, SL>(p, stream);
  if (p.d <= 32) return dispatch_f32_mt<2, SL>(p, stream);
  if (p.d <= 64) return dispatch_f32_mt<4, SL>(p, stream);
  return dispatch_f32_mt<8, SL>(p, stream);
}

}  // namespace

int launch_based_parallel_fp32(const ParallelArgs& a, hipStream_t stream) {
  F32Params p{};
  p.q = static_cast<const float*>(a.q);
  p.k = static_cast<const float*>(a.k);
  p.v = static_cast<const float*>(a.v);
  p.out = a.out;
  p.den = a.den;
  p.BH = a.BH;
  p.N = a.N;
  p.d = a.d;
  p.dv = a.dv;
  const float icf = (float)(1.0 / (double)a.scale);
  p.inv_c = icf;
  p.inv_c2 = (float)((double)icf * (double)icf);
  p.fscale = (float)(1.0 / (2.0 * (double)icf * (double)icf));
  p.eps = a.eps;
  p.normalize = a.normalize ? 1 : 0;
  p.out_f32 = a.out_f32 ? 1 : 0;
  return dispatch_f32<false>(p, stream);
}

int launch_sliding_window_f32(const SlidingArgs& a, hipStream_t stream) {
  F32Params p{};
  p.q = static_cast<const float*>(a.q);
  p.k = static_cast<const float*>(a.k);
  p.v = static_cast<const float*>(a.v);
  p.out = a.out;
  p.addend = a.addend;
  p.BH = a.BH;
  p.N = a.N;
  p.d = a.d;
  p.dv = a.dv;
  p.window = a.window;
  p.scale_log2 = (float)((double)a.scale * 1.4426950408889634);
  p.out_f32 = a.out_f32 ? 1 : 0;
  return dispatch_f32<true>(p, stream);
}

}  // namespace la
