// One recurrent (decode) step of BASED causal linear attention for gfx950, on the state the
// chunked kernel exports: per head the fp32 (F x (dv + 1)) matrix [S | z] with
// S = sum_u phi(k_u) v_u^T and z = sum_u phi(k_u) over the tokens so far, phi the Taylor
// feature map of benchmarks/chunked_attention_benchmark.py:34-53 in its order
//   phi(x) = [1, x_i / d^(1/4), x_i^2 / (sqrt(d) sqrt(2)), x_i x_j / sqrt(d) (i < j, row-major)],
// F = 1 + d + d(d+1)/2, so that phi(q).phi(k) = 1 + s + s^2/2 with s = q.k / sqrt(d).
// For the new token (q, k, v) of every head the step does
//   [S | z] += phi(k) [v | 1],   num = phi(q)^T [S | z],   y = num[:dv] / (num[dv] + eps)
// which is the chunk recurrence of kernels/nki_attention_chunked.py:65-109 for a chunk of one
// token (its intra-chunk term phi(q).phi(k) v is the contribution of the token's own row of the
// update).  The reference has no decode path; this continues a prefill that exported its state.
//
// A head whose state fits in LDS (F (dv + 1) <= 10240 floats) runs in one 1024-thread
// work-group that loads the whole state at once (based_decode_wide_kernel).  Otherwise a
// head's F state rows are split into R groups of consecutive rows, one work-group each: phi(q)
// and phi(k) of the group's rows go to LDS, then the group's rows are swept linearly
// (coalesced) in tiles of 32 rows, each element updated in place, and the column sums of phi(q)
// times the updated state are taken per tile through LDS in row order.  With R = 1 the
// work-group normalises and stores the output itself; with R > 1 it stores its column sums to
// a workspace and a combine kernel adds the R partial sums of every column in group order
// (deterministic) and normalises.  R is chosen so that small batches still launch enough
// work-groups to cover the chip.  HBM-bound: the state is read and written once
// (4 F (dv + 1) bytes each way per head).
#include <math.h>

#include <algorithm>

#include "la_common.hpp"
#include "la_internal.hpp"

namespace la {

namespace {

struct DecodeParams {
  const void* q;
  const void* k;
  const void* v;
  float* state;
  void* out;
  int BH, d, dv, F;
  float eps;
  int normalize, in_f32, out_f32;
};

constexpr int kDecThreads = 256;
constexpr int kDecMaxD = 64;
constexpr int kDecMaxC = 129;   // dv + 1 for dv <= 128
constexpr int kDecMaxF = 1 + kDecMaxD + kDecMaxD * (kDecMaxD + 1) / 2;
constexpr int kDecRows = 32;    // state rows per reduction tile
constexpr int kDecMinRows = 8;  // fewest state rows per work-group when a head is split
constexpr int kWideThreads = 1024;
constexpr int kWideMaxElems = 10240;   // F (dv + 1) state floats of one head held in LDS (40 KB)
constexpr int kWidePer = kWideMaxElems / kWideThreads;
#ifndef LA_DECODE_TARGET_WGS
#define LA_DECODE_TARGET_WGS 1024   // split heads until about this many work-groups launch
#endif

__device__ __forceinline__ float load_elem(const void* base, size_t i, bool f32) {
  return f32 ? static_cast<const float*>(base)[i] : bf16_bits_to_f32(static_cast<const uint16_t*>(base)[i]);
}

// Feature f of phi(x) (reference order), x in LDS.
__device__ __forceinline__ float feature(const float* x, int f, int d, float r4, float rsq, float rd) {
  if (f == 0) return 1.f;
  if (f <= d) return x[f - 1] * r4;
  if (f <= 2 * d) {
    const float t = x[f - 1 - d];
    return t * t * rsq;
  }
  int t = f - 1 - 2 * d, i = 0;
  while (t >= d - 1 - i) {   // row i of the strict upper triangle holds d - 1 - i pairs
    t -= d - 1 - i;
    ++i;
  }
  return x[i] * x[i + 1 + t] * rd;
}

// Rows [g RW, min(F, (g + 1) RW)) of head bh = blockIdx.x, g = blockIdx.y.  PARTIAL: store
// the group's column sums to part[(bh R + g) C + c]; else (R = 1) normalise and store the output.
template <bool PARTIAL>
__global__ __launch_bounds__(kDecThreads) void based_decode_kernel(const DecodeParams p, int RW, float* part) {
  __shared__ float xq[kDecMaxD], xk[kDecMaxD], vv[kDecMaxC];
  __shared__ float phq[kDecMaxF], phk[kDecMaxF];
  __shared__ float tile[kDecRows * kDecMaxC];
  const int bh = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
  const int d = p.d, dv = p.dv, F = p.F, C = dv + 1;
  const int rb = g * RW, re = min(F, rb + RW);
  if (tid < d) {
    xq[tid] = load_elem(p.q, (size_t)bh * d + tid, p.in_f32);
    xk[tid] = load_elem(p.k, (size_t)bh * d + tid, p.in_f32);
  }
  if (tid < dv) vv[tid] = load_elem(p.v, (size_t)bh * dv + tid, p.in_f32);
  if (tid == 0) vv[dv] = 1.f;
  __syncthreads();
  const float rd = 1.0f / sqrtf((float)d), r4 = sqrtf(rd), rsq = rd * 0.70710678118654752f;
  for (int f = rb + tid; f < re; f += kDecThreads) {
    phq[f - rb] = feature(xq, f, d, r4, rsq, rd);
    phk[f - rb] = feature(xk, f, d, r4, rsq, rd);
  }
  __syncthreads();

  // The rows sweep linearly (coalesced) in tiles of kDecRows rows: every element is updated in
  // place and its phi(q)-weighted value parked in LDS, then thread c < C adds the tile's column
  // c in row order.
  float* __restrict__ st = p.state + (size_t)bh * F * C;
  float colsum = 0.f;
  for (int r0 = rb; r0 < re; r0 += kDecRows) {
    const int ne = min(kDecRows, re - r0) * C;
    float* __restrict__ base = st + (size_t)r0 * C;
    const float* pk = phk + (r0 - rb);
    const float* pq = phq + (r0 - rb);
    for (int e = tid; e < ne; e += kDecThreads) {
      const int fr = e / C, c = e - fr * C;
      const float s = __builtin_fmaf(pk[fr], vv[c], base[e]);
      base[e] = s;
      tile[e] = pq[fr] * s;
    }
    __syncthreads();
    if (tid < C)
      for (int e = tid; e < ne; e += C) colsum += tile[e];
    __syncthreads();
  }
  if (PARTIAL) {
    if (tid < C) part[((size_t)bh * gridDim.y + g) * C + tid] = colsum;
    return;
  }
  __shared__ float den;
  if (tid == dv) den = colsum;
  __syncthreads();
  if (tid < dv) {
    const float y = p.normalize ? colsum / (den + p.eps) : colsum;
    const size_t o = (size_t)bh * dv + tid;
    if (p.out_f32)
      static_cast<float*>(p.out)[o] = y;
    else
      static_cast<uint16_t*>(p.out)[o] = f32_to_bf16_bits(y);
  }
}

// Heads whose whole state fits in LDS (F (dv + 1) <= kWideMaxElems): one work-group of
// kWideThreads per head.  Every state element of the head is loaded at the start (one memory
// latency instead of one per tile), updated in place, and its phi(q)-weighted value parked in
// LDS; thread (segment, c) then adds rows [segment RS, (segment + 1) RS) of column c in row order
// and thread c adds the segments in order (deterministic).
__global__ __launch_bounds__(kWideThreads) void based_decode_wide_kernel(const DecodeParams p) {
  __shared__ float xq[kDecMaxD], xk[kDecMaxD], vv[kDecMaxC];
  __shared__ float phq[kDecMaxF], phk[kDecMaxF];
  __shared__ float tile[kWideMaxElems];
  __shared__ float part[kWideThreads];
  __shared__ float den;
  const int bh = blockIdx.x, tid = threadIdx.x;
  const int d = p.d, dv = p.dv, F = p.F, C = dv + 1, FC = F * C;
  float* __restrict__ st = p.state + (size_t)bh * FC;
  float pre[kWidePer];
#pragma unroll
  for (int i = 0; i < kWidePer; ++i) {
    const int e = tid + kWideThreads * i;
    pre[i] = e < FC ? st[e] : 0.f;
  }
  if (tid < d) {
    xq[tid] = load_elem(p.q, (size_t)bh * d + tid, p.in_f32);
    xk[tid] = load_elem(p.k, (size_t)bh * d + tid, p.in_f32);
  }
  if (tid < dv) vv[tid] = load_elem(p.v, (size_t)bh * dv + tid, p.in_f32);
  if (tid == 0) vv[dv] = 1.f;
  __syncthreads();
  const float rd = 1.0f / sqrtf((float)d), r4 = sqrtf(rd), rsq = rd * 0.70710678118654752f;
  for (int f = tid; f < F; f += kWideThreads) {
    phq[f] = feature(xq, f, d, r4, rsq, rd);
    phk[f] = feature(xk, f, d, r4, rsq, rd);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kWidePer; ++i) {
    const int e = tid + kWideThreads * i;
    if (e < FC) {
      const int fr = e / C, c = e - fr * C;
      const float s = __builtin_fmaf(phk[fr], vv[c], pre[i]);
      st[e] = s;
      tile[e] = phq[fr] * s;
    }
  }
  __syncthreads();
  const int NS = kWideThreads / C, RS = (F + NS - 1) / NS;
  const int seg = tid / C, col = tid - seg * C;
  if (seg < NS) {
    float r = 0.f;
    const int r1 = min(F, (seg + 1) * RS);
    for (int f = seg * RS; f < r1; ++f) r += tile[f * C + col];
    part[seg * C + col] = r;
  }
  __syncthreads();
  float colsum = 0.f;
  if (tid < C)
    for (int sg = 0; sg < NS; ++sg) colsum += part[sg * C + tid];
  if (tid == dv) den = colsum;
  __syncthreads();
  if (tid < dv) {
    const float y = p.normalize ? colsum / (den + p.eps) : colsum;
    const size_t o = (size_t)bh * dv + tid;
    if (p.out_f32)
      static_cast<float*>(p.out)[o] = y;
    else
      static_cast<uint16_t*>(p.out)[o] = f32_to_bf16_bits(y);
  }
}

// Head bh = blockIdx.x: column c = sum over groups g = 0 .. R-1 (in that order) of
// part[(bh R + g) C + c], then the output as in the single-group kernel.
__global__ __launch_bounds__(kDecThreads) void decode_combine_kernel(const DecodeParams p, int R,
                                                                     const float* __restrict__ part) {
  __shared__ float den;
  const int bh = blockIdx.x, tid = threadIdx.x, dv = p.dv, C = dv + 1;
  float colsum = 0.f;
  if (tid < C) {
    // eight loads in flight at a time; the additions keep group order
    const float* src = part + (size_t)bh * R * C + tid;
    int g = 0;
    for (; g + 8 <= R; g += 8) {
      float t[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) t[i] = src[(size_t)(g + i) * C];
#pragma unroll
      for (int i = 0; i < 8; ++i) colsum += t[i];
    }
    for (; g < R; ++g) colsum += src[(size_t)g * C];
  }
  if (tid == dv) den = colsum;
  __syncthreads();
  if (tid < dv) {
    const float y = p.normalize ? colsum / (den + p.eps) : colsum;
    const size_t o = (size_t)bh * dv + tid;
    if (p.out_f32)
      static_cast<float*>(p.out)[o] = y;
    else
      static_cast<uint16_t*>(p.out)[o] = f32_to_bf16_bits(y);
  }
}

}  // namespace

bool decode_shape(int d, int dv) { return d >= 1 && d <= kDecMaxD && dv >= 1 && dv + 1 <= kDecMaxC; }

// Row groups per head: enough work-groups for the chip, at least kDecMinRows rows each; RW =
// rows per group (the last group may have fewer).
static void decode_groups(long long BH, int d, int& R, int& RW) {
  const int F = 1 + d + d * (d + 1) / 2;
  long long r = (LA_DECODE_TARGET_WGS + BH - 1) / BH;
  r = std::max(1LL, std::min(r, (long long)((F + kDecMinRows - 1) / kDecMinRows)));
  RW = (int)((F + r - 1) / r);
  R = (F + RW - 1) / RW;
}

static bool decode_wide(int d, int dv) { return (1 + d + d * (d + 1) / 2) * (dv + 1) <= kWideMaxElems; }

size_t decode_workspace_bytes(long long BH, int d, int dv) {
  if (decode_wide(d, dv)) return 0;
  int R, RW;
  decode_groups(BH, d, R, RW);
  return R > 1 ? (size_t)BH * R * (dv + 1) * sizeof(float) : 0;
}

int launch_decode_step(const DecodeArgs& a, hipStream_t stream) {
  DecodeParams p{};
  p.q = a.q;
  p.k = a.k;
  p.v = a.v;
  p.state = a.state;
  p.out = a.out;
  p.BH = a.BH;
  p.d = a.d;
  p.dv = a.dv;
  p.F = 1 + a.d + a.d * (a.d + 1) / 2;
  p.eps = a.eps;
  p.normalize = a.normalize ? 1 : 0;
  p.in_f32 = a.in_f32 ? 1 : 0;
  p.out_f32 = a.out_f32 ? 1 : 0;
  if (decode_wide(a.d, a.dv)) {
    hipLaunchKernelGGL(based_decode_wide_kernel, dim3((unsigned)a.BH), dim3(kWideThreads), 0, stream, p);
    return (int)hipGetLastError();
  }
  int R = 1, RW = p.F;
  if (a.workspace != nullptr) decode_groups(a.BH, a.d, R, RW);
  if (R == 1) {
    hipLaunchKernelGGL(based_decode_kernel<false>, dim3((unsigned)a.BH, 1), dim3(kDecThreads), 0, stream, p, RW,
                       static_cast<float*>(nullptr));
  } else {
    float* part = static_cast<float*>(a.workspace);
    hipLaunchKernelGGL(based_decode_kernel<true>, dim3((unsigned)a.BH, (unsigned)R), dim3(kDecThreads), 0, stream,
                       p, RW, part);
    hipLaunchKernelGGL(decode_combine_kernel, dim3((unsigned)a.BH), dim3(kDecThreads), 0, stream, p, R,
                       static_cast<const float*>(part));
  }
  return (int)hipGetLastError();
}

}  // namespace la
