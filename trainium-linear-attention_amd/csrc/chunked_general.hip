// Chunked BASED attention for head dims other than the d = 16 kernel's: any d <= 64 and
// dv <= 128, bf16 inputs.  Linear in N: the sequence is cut into segments of GL tokens; the
// tokens of a segment see the earlier segments through their state and each other through the
// quadratic form, as the chunk recurrence of kernels/nki_attention_chunked.py:65-109 with
// chunk = GL (the recurrence gives the same function for every chunk size).  The feature basis
// (block-symmetric groups over [k, 1]) is described in la_general.hpp.
//
// Kernel 0 (gprep_kernel) converts every 64-token chunk before the last segment once: per-token
// normalised fp16 k~^T rows, v n^2 rows and the n^2 row with the chunk's exponents.
// Kernel 1 (gstate_kernel): one work-group per (head, 16 groups); its eight waves hold one
// 32-feature tile each as fp32 MFMA accumulators over dv and sweep the head's converted chunks
// through an LDS ring (buffer_load ... lds, NS - 1 chunks ahead): A = feature rows (one
// v_pk_mul_f16 per two products k~_i k~_j), B = the V^T rows, K = tokens, fp16 MFMAs; z from the
// same products against the n^2 row.  After every segment but the last it writes the state so
// far, the exclusive prefix of the next segment, as fp16 with one exponent per (segment,
// work-group).
// Kernel 2 (gout_kernel): one work-group per 256 queries (four waves of 64).  The inter-segment
// part is O^T += T^T Phi(Q)^T over all groups on fp16 MFMAs: T^T blocks of 4 groups copied into
// LDS (buffer_load ... lds, three blocks in flight), Phi(Q) formed in registers from the query's
// features a'/m (m a power of two >= max |a'|, so every feature lies in [-1, 1]) with one
// v_pk_mul_f16 per two features; the per-group weight times 2^(E_tile - E_max) goes on a'_i.
// The denominator takes the same features against z with v_dot2.  The intra-segment part is the
// quadratic form over the segment's keys up to the query (bf16 score MFMAs, p in fp32, P.V as two
// bf16 MFMAs on p's hi and lo parts), added before the division.
#include <float.h>

#include "../../include/based_la.h"
#include "la_common.hpp"
#include "la_general.hpp"
#include "la_internal.hpp"
#include "la_stage.hpp"

namespace la {
namespace {

struct GParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  void* out;
  uint16_t* T;      // [seg-1][BH][NGB][DVP rows][64] fp16, 16-byte unit u of a row at u ^ ((row >> 1) & 7)
  uint16_t* Z;      // [seg-1][BH][NGB * 64] fp16
  int* E;           // [seg-1][BH][NWGA]
  uint16_t* KV;     // converted chunks [BH][chunks before the last segment][GChunk rows][64]
  u32x2* CE;        // their exponents {Ec, Ez}
  float* Tot;       // per (part < nparts - 1, head, state work-group, thread): its part's sums
  u32* VM;          // [BH][kVmParts] partial maxima of |v| (bf16 bits) over the prefix tokens
  float* den_out;   // optional (BH, N): each row's denominator without eps
  int nparts, spp;  // the state sweep split into parts of spp segments
  int BH, N, d, dv, nseg, vec;
  float scale, eps;
  int normalize, out_f32;
  int alt_prio;     // state kernel: more work-groups than CUs (two share a CU), alternate priorities
};

constexpr u32 kOnesBf16 = 0x3f803f80u;

// Wait until at most n of this wave's vector-memory operations are outstanding (s_waitcnt
// vmcnt(n), n <= 31; lgkmcnt and expcnt untouched).
__device__ __forceinline__ void wait_vm(int n) {
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

// Rows of a converted 64-token chunk (fp16, 128 bytes each): k~^T rows 0 .. DP (row DP the
// augmented 1/n), V^T rows, one row of n^2, a row holding the chunk's exponents, zero rows up
// to a multiple of 8.  The exponents travel with the rows, so that the state kernel reads them
// from LDS with the chunk.  The eight 16-byte
// units of row r are stored XOR ((r >> 1) & 7), which makes the 16-row fragment reads of a lane
// group conflict-free.
template <int DP, int DVT>
struct GChunk {
  static constexpr int DVP = 32 * DVT;
  static constexpr int RV = DP + 1;             // first V^T row
  static constexpr int RN = DP + 1 + DVP;       // the n^2 row
  static constexpr int RE = RN + 1;             // the chunk's exponents {Ec, Ez} (two int32)
  static constexpr int ROWS = (RE + 1 + 7) & ~7;
  static constexpr int HALVES = ROWS * GC;
  static constexpr int UNITS = ROWS / 8;        // 1 KB copy units
};

__device__ __forceinline__ int gswz(int row, int unit) { return (unit ^ ((row >> 1) & 7)) << 3; }

// ---------------------------------------------------------------- head V exponent
// The prefixes T hold sums of phi(k) v in fp16 beside z = sums of phi(k) with one exponent per
// (segment, work-group), so V enters them divided by 2^Eh, Eh = floor(log2 max |v|) over the
// head's tokens before its last segment (the ones the prefixes sum): then T and z keep
// comparable magnitudes for V of any size (without it, T of a head with |v| ~ 1e-20 would flush
// to zero beside z), and the output kernel multiplies the inter-segment numerator by 2^Eh.
constexpr int kVmParts = 64;

// Work-group (part, head): the largest |v| (bf16 bits) of its share of the prefix tokens.
__global__ __launch_bounds__(256) void gvmax_kernel(const GParams p) {
  __shared__ u32 wm[4];
  const int tid = threadIdx.x, s = blockIdx.x, bh = blockIdx.y;
  const int R = (p.nseg - 1) * GL;                        // prefix tokens (< N)
  const int per = (R + kVmParts - 1) / kVmParts;
  const int r0 = min(R, s * per), r1 = min(R, r0 + per);
  const uint16_t* base = p.v + ((size_t)bh * p.N + r0) * p.dv;
  const long long n = (long long)(r1 - r0) * p.dv;
  u32 m = 0u;
  long long i0 = 0;
  if ((reinterpret_cast<uintptr_t>(base) & 15) == 0) {   // 16-byte loads over the whole units
    const u32x4* b4 = reinterpret_cast<const u32x4*>(base);
    const long long n8 = n / 8;
    for (long long i = tid; i < n8; i += 256) {
      const u32x4 x = b4[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) m = max(m, max(x[e] & 0x7fffu, (x[e] >> 16) & 0x7fffu));
    }
    i0 = n8 * 8;
  }
  for (long long i = i0 + tid; i < n; i += 256) m = max(m, (u32)(base[i] & 0x7fffu));
  m = wave_max_u32(m);
  if ((tid & 63) == 0) wm[tid >> 6] = m;
  __syncthreads();
  if (tid == 0) p.VM[(size_t)bh * kVmParts + s] = max(max(wm[0], wm[1]), max(wm[2], wm[3]));
}

// Eh of head bh from its partial maxima (every lane of the wave calls it; the result is uniform).
__device__ __forceinline__ int head_vexp(const GParams& p, int bh) {
  const int lane = threadIdx.x & 63;
  const u32 m = wave_max_u32(p.VM[(size_t)bh * kVmParts + lane]);
  return m == 0u ? 0 : (int)((m << 16) >> 23) - 127;   // bf16 subnormals: -127
}

// ---------------------------------------------------------------- kernel 0: chunk conversion
// One work-group per (head, 64-token chunk) of the tokens before the last segment.  Per token t:
// n_t = 2^e >= max(max_i |k_ti|, 1), k~ = [k, 1] / n_t in fp16 (every entry in [-1, 1]); the
// token's features are then phi(k~) = phi([k, 1]) / n_t^2, so the V^T rows carry v n_t^2 and the
// z row n_t^2, each scaled by a power of two of the chunk (Ec, Ez, multiples of 8: the chunk's
// largest value in [2^7, 2^15)), written to CE[head][chunk] = {Ec, Ez}.
template <int DP, int DVT>
__global__ __launch_bounds__(256) void gprep_kernel(const GParams p) {
  using CK = GChunk<DP, DVT>;
  constexpr int DVP = CK::DVP, KPP = DP / 4, VPP = DVP / 4;
  __shared__ __attribute__((aligned(16))) uint16_t blk[CK::HALVES];
  __shared__ u32 red[2][4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nch = (p.nseg - 1) * (GL / GC);
  const int bh = blockIdx.x / nch, c = blockIdx.x - bh * nch;
  const int N = p.N, d = p.d, dv = p.dv;
  const int t = tid >> 2, part = tid & 3;
  const size_t row = (size_t)bh * N + (size_t)c * GC + t;   // inside the sequence: c < nch

  float kv[KPP], vv[VPP];
  if (p.vec) {
    // 16-byte rows of k (d % 8 == 0) and 8-byte groups of v (dv % 4 == 0)
#pragma unroll
    for (int e = 0; e < KPP; e += 4) {
      const int col = part * KPP + e;
      const u32x2 x = col < d ? *reinterpret_cast<const u32x2*>(p.k + row * d + col) : (u32x2){0u, 0u};
      kv[e] = bf16_lo_to_f32(x[0]);
      kv[e + 1] = bf16_hi_to_f32(x[0]);
      kv[e + 2] = bf16_lo_to_f32(x[1]);
      kv[e + 3] = bf16_hi_to_f32(x[1]);
    }
#pragma unroll
    for (int e = 0; e < VPP; e += 4) {
      const int col = part * VPP + e;
      const u32x2 x = col < dv ? *reinterpret_cast<const u32x2*>(p.v + row * dv + col) : (u32x2){0u, 0u};
      vv[e] = bf16_lo_to_f32(x[0]);
      vv[e + 1] = bf16_hi_to_f32(x[0]);
      vv[e + 2] = bf16_lo_to_f32(x[1]);
      vv[e + 3] = bf16_hi_to_f32(x[1]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < KPP; ++e) {
      const int col = part * KPP + e;
      kv[e] = col < d ? bf16_bits_to_f32(p.k[row * d + col]) : 0.f;
    }
#pragma unroll
    for (int e = 0; e < VPP; ++e) {
      const int col = part * VPP + e;
      vv[e] = col < dv ? bf16_bits_to_f32(p.v[row * dv + col]) : 0.f;
    }
  }
  {
    const int eh = head_vexp(p, bh);   // V / 2^Eh (exact)
#pragma unroll
    for (int e = 0; e < VPP; ++e) vv[e] = __builtin_ldexpf(vv[e], -eh);
  }
  u32 mk = 0u, mv = 0u;
#pragma unroll
  for (int e = 0; e < KPP; ++e) mk = max(mk, __builtin_bit_cast(u32, __builtin_fabsf(kv[e])));
#pragma unroll
  for (int e = 0; e < VPP; ++e) mv = max(mv, __builtin_bit_cast(u32, __builtin_fabsf(vv[e])));
  // the token's four parts are lanes 4t .. 4t+3
  mk = max(mk, (u32)__shfl_xor((int)mk, 1));
  mk = max(mk, (u32)__shfl_xor((int)mk, 2));
  mv = max(mv, (u32)__shfl_xor((int)mv, 1));
  mv = max(mv, (u32)__shfl_xor((int)mv, 2));
  int en;
  (void)__builtin_frexpf(__builtin_fmaxf(__builtin_bit_cast(float, mk), 1.0f), &en);
  const float inv = __builtin_ldexpf(1.0f, -en);
  // chunk maxima of |v| n^2 and n^2
  const float vn = __builtin_ldexpf(__builtin_bit_cast(float, mv), 2 * en);
  u32 cv = wave_max_u32(__builtin_bit_cast(u32, vn));
  u32 cz = wave_max_u32((u32)en);
  if (lane == 0) {
    red[0][w] = cv;
    red[1][w] = cz;
  }
  __syncthreads();
  cv = max(max(red[0][0], red[0][1]), max(red[0][2], red[0][3]));
  cz = max(max(red[1][0], red[1][1]), max(red[1][2], red[1][3]));
  // exponents in steps of 8 (largest value in [2^7, 2^15)), so that chunks of one order of
  // magnitude share them and the state kernel scales nothing
  const int ev = cv == 0u ? -1000 : (int)(cv >> 23) - 127;   // chunk max of |v| n^2 in [2^ev, 2^(ev+1))
  const int Ec = cv == 0u ? 0 : 8 * ((ev - 14 + 7 + 1024) / 8 - 128);
  const int Ez = 8 * ((2 * (int)cz - 1 - 14 + 7 + 1024) / 8 - 128);
  const float sv = __builtin_ldexpf(1.0f, 2 * en - Ec), sz = __builtin_ldexpf(1.0f, 2 * en - Ez);

  // rows into LDS, [row][64 tokens] unswizzled
#pragma unroll
  for (int e = 0; e < KPP; ++e) blk[(part * KPP + e) * GC + t] = (uint16_t)(pack_f16x2(kv[e] * inv, 0.f) & 0xffffu);
#pragma unroll
  for (int e = 0; e < VPP; ++e) blk[(CK::RV + part * VPP + e) * GC + t] = (uint16_t)(pack_f16x2(vv[e] * sv, 0.f) & 0xffffu);
  if (part == 0) {
    blk[DP * GC + t] = (uint16_t)(pack_f16x2(inv, 0.f) & 0xffffu);
    blk[CK::RN * GC + t] = (uint16_t)(pack_f16x2(sz, 0.f) & 0xffffu);
  }
  for (int x = tid; x < (CK::ROWS - CK::RE) * GC; x += 256) blk[CK::RE * GC + x] = 0;
  __syncthreads();
  if (tid == 0) *reinterpret_cast<u32x2*>(&blk[CK::RE * GC]) = (u32x2){(u32)Ec, (u32)Ez};
  __syncthreads();
  // out: 16-byte units, swizzled within each row
  uint16_t* dst = p.KV + ((size_t)bh * nch + c) * CK::HALVES;
  for (int u = tid; u < CK::ROWS * 8; u += 256) {
    const int r = u >> 3, x = u & 7;
    *reinterpret_cast<u32x4*>(dst + r * GC + gswz(r, x)) = *reinterpret_cast<const u32x4*>(&blk[r * GC + 8 * x]);
  }
  if (tid == 0) p.CE[(size_t)bh * nch + c] = (u32x2){(u32)Ec, (u32)Ez};
}

// ---------------------------------------------------------------- kernel 1: segment states
// Sequences with few heads split the sweep into p.nparts parts of p.spp segments: a TOTAL pass
// sums every part but the last (no prefixes written), then each part's work-group starts from
// the totals of the parts before it and writes its segments' prefixes.  The work-group's eight
// 32-feature tiles go to 8 / TW waves of TW tiles each.
template <int DP, int DVT, bool TOTAL, int TW>
__global__ __launch_bounds__(64 * (8 / TW), TW == 1 ? 4 : 1) void gstate_kernel(const GParams p) {
  using FT = GFeat<DP>;
  using CK = GChunk<DP, DVT>;
  constexpr int NWV = 8 / TW, NT = 64 * NWV;
  constexpr int DVP = CK::DVP, NS = DVT == 4 ? 3 : 4;   // ring stages (prefetch distance NS - 1)
  // a stage: the chunk's rows, then 16 zero rows standing for k~^T rows DP + 1 .. DP + 16
  constexpr int SH = CK::HALVES + 16 * GC;
  __shared__ __attribute__((aligned(16))) uint16_t ring[NS][SH];
  __shared__ u32 red[3][NWV];
  auto red_max = [&](int row) {
    u32 m = red[row][0];
#pragma unroll
    for (int i = 1; i < NWV; ++i) m = max(m, red[row][i]);
    return m;
  };

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
  const int nch = (p.nseg - 1) * (GL / GC);
  const int cps = GL / GC;
  const int c0 = part * p.spp * cps, c1 = min((part + 1) * p.spp, p.nseg - 1) * cps;   // this part's chunks
  constexpr int PER = TW * (DVT * 16 + 1);   // a thread's sums: accumulators, then z partials
  const uint16_t* __restrict__ src = p.KV + (size_t)bh * nch * CK::HALVES;
  const u32x2* __restrict__ ce = p.CE + (size_t)bh * nch;

  for (int x = tid; x < NS * 16 * GC; x += NT) ring[x / (16 * GC)][CK::HALVES + x % (16 * GC)] = 0;

  // the head's reference exponents: the largest chunk exponents
  u32 mc = 0u, mz = 0u;   // biased by 1024 so that the unsigned maximum orders them
  for (int c = tid; c < nch; c += NT) {
    const u32x2 e2 = ce[c];
    mc = max(mc, (u32)((int)e2[0] + 1024));
    mz = max(mz, (u32)((int)e2[1] + 1024));
  }
  mc = wave_max_u32(mc);
  mz = wave_max_u32(mz);
  if (lane == 0) {
    red[0][w] = mc;
    red[1][w] = mz;
  }

  // this lane's feature rows of its tiles: k~^T row i (<= DP) and row j (> DP: a zero row of
  // the stage).  A wave whose tile lies past the last one computes group 0 and stores nothing.
  int ri[TW], rj[TW], xi[TW], xj[TW];
  bool tv[TW];
#pragma unroll
  for (int mw = 0; mw < TW; ++mw) {
    const int tt = 8 * wga + TW * w + mw;
    tv[mw] = tt < FT::NT;
    int i, J;
    group_ij<DP>(tv[mw] ? 2 * tt + (n >> 4) : 0, i, J);
    const int j = 16 * J + (n & 15);
    ri[mw] = i;
    xi[mw] = (i >> 1) & 7;
    rj[mw] = j > DP ? CK::ROWS + (j - DP - 1) : j;
    xj[mw] = (rj[mw] >> 1) & 7;
  }
  int rv[DVT];
#pragma unroll
  for (int nt = 0; nt < DVT; ++nt) rv[nt] = CK::RV + 32 * nt + n;

  constexpr int UW = (CK::UNITS + NWV - 1) / NWV;   // most copy units per wave and chunk
  const int my_units = CK::UNITS / NWV + (w < CK::UNITS % NWV ? 1 : 0);
  const u32x4 rsrc = buffer_rsrc(src, (u32)((size_t)nch * CK::HALVES * 2));
  auto issue = [&](int c) {
    if (c >= c1) return;
    const u32 base = lds_addr(&ring[c % NS][0]);
#pragma unroll
    for (int x = 0; x < UW; ++x) {
      const int u = w + NWV * x;
      if (u < CK::UNITS) lds_copy16(rsrc, base + 1024 * u, c * (CK::HALVES * 2) + 1024 * u + 16 * lane);
    }
  };
  __syncthreads();
  const int eref = (int)red_max(0) - 1024;
  const int ezref = (int)red_max(1) - 1024;

  f32x16 acc[TW][DVT];
  float zc[TW];
#pragma unroll
  for (int mw = 0; mw < TW; ++mw) zc[mw] = 0.f;
#pragma unroll
  for (int mw = 0; mw < TW; ++mw)
#pragma unroll
    for (int nt = 0; nt < DVT; ++nt) acc[mw][nt] = splat16(0.f);

  if (!TOTAL) {
    // the parts before this one
    for (int q = 0; q < part; ++q) {
      const float* t = p.Tot + (((size_t)q * p.BH + bh) * nwga + wga) * (NT * PER) + tid * PER;
#pragma unroll
      for (int mw = 0; mw < TW; ++mw) {
#pragma unroll
        for (int nt = 0; nt < DVT; ++nt)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[mw][nt][r] += t[(mw * DVT + nt) * 16 + r];
        zc[mw] += t[TW * DVT * 16 + mw];
      }
    }
  }
  for (int c = c0; c < c0 + NS - 1; ++c) issue(c);
  for (int gc = c0; gc < c1; ++gc) {
    // Of two work-groups on one CU the older one's waves issue first at equal priority and the
    // younger one fell behind, then ran alone.  Priority 1 at even chunks and 0 at odd ones
    // alternates the lead, so their progress stays within about a chunk (B2 H16 N8192 d64
    // 444 -> 424 us, N16384 886 -> 863 us in one process; no change where each CU holds one).
    if (p.alt_prio) {
      if ((gc - c0) & 1)
        __builtin_amdgcn_s_setprio(0);
      else
        __builtin_amdgcn_s_setprio(1);
    }
    // this wave's copies of chunk gc landed (later chunks may still be in flight), then every
    // wave's; every wave is also done with chunk gc - 1, whose stage the next copy reuses
    wait_vm(my_units * min(NS - 2, c1 - 1 - gc));
    __syncthreads();
    issue(gc + NS - 1);
    const uint16_t* st = &ring[gc % NS][0];
    const u32x2 e2 = *reinterpret_cast<const u32x2*>(st + CK::RE * GC + gswz(CK::RE, 0));
    const int dc = (int)e2[0] - eref, dz = (int)e2[1] - ezref;
    // the chunk's V^T and n^2 rows in the head's units (multiplied by 2^dc, 2^dz <= 1): only for
    // chunks whose exponents are below the head's
    const bool scaled = (dc | dz) != 0;
    const u32 fkp = scaled ? pack_f16x2(__builtin_ldexpf(1.0f, dc), __builtin_ldexpf(1.0f, dc)) : 0x3c003c00u;
    const u32 fzp = scaled ? pack_f16x2(__builtin_ldexpf(1.0f, dz), __builtin_ldexpf(1.0f, dz)) : 0x3c003c00u;
    auto kstep = [&](int ks, bool sc) {
      const int u = 2 * ks + h;
      u32x4 vf[DVT];
#pragma unroll
      for (int nt = 0; nt < DVT; ++nt) {
        vf[nt] = *reinterpret_cast<const u32x4*>(st + rv[nt] * GC + gswz(rv[nt], u));
        if (sc)
#pragma unroll
          for (int c4 = 0; c4 < 4; ++c4) vf[nt][c4] = pk_mul_f16(vf[nt][c4], fkp);
      }
      u32x4 nz = *reinterpret_cast<const u32x4*>(st + CK::RN * GC + gswz(CK::RN, u));
      if (sc)
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) nz[c4] = pk_mul_f16(nz[c4], fzp);
      u32x4 bi[TW], bj[TW];
#pragma unroll
      for (int mw = 0; mw < TW; ++mw) {
        bi[mw] = *reinterpret_cast<const u32x4*>(st + ri[mw] * GC + ((u ^ xi[mw]) << 3));
        bj[mw] = *reinterpret_cast<const u32x4*>(st + rj[mw] * GC + ((u ^ xj[mw]) << 3));
      }
#pragma unroll
      for (int mw = 0; mw < TW; ++mw) {
        const u32x4 af = {pk_mul_f16(bi[mw][0], bj[mw][0]), pk_mul_f16(bi[mw][1], bj[mw][1]),
                          pk_mul_f16(bi[mw][2], bj[mw][2]), pk_mul_f16(bi[mw][3], bj[mw][3])};
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) zc[mw] = dot2_f16(af[c4], nz[c4], zc[mw]);
#pragma unroll
        for (int nt = 0; nt < DVT; ++nt) acc[mw][nt] = mfma32x32x16_f16(af, vf[nt], acc[mw][nt]);
      }
    };
    // one K step at a time on one-tile waves (the 128-VGPR budget), all of them unrolled on two
    constexpr int KSU = TW == 1 ? 1 : GC / 16;
    if (scaled) {
#pragma unroll KSU
      for (int ks = 0; ks < GC / 16; ++ks) kstep(ks, true);
    } else {
#pragma unroll KSU
      for (int ks = 0; ks < GC / 16; ++ks) kstep(ks, false);
    }

    if (!TOTAL && (gc + 1) % cps == 0) {
      // end of segment s = gc / cps: write the prefix of segment s + 1 (slot s).  acc holds
      // T 2^-eref, zc z 2^-ezref; the slot's exponent E puts the largest of both in
      // [2^13, 2^14).
      const int s = gc / cps;
      float zz[TW];
      u32 ma = 0u, mzz = 0u;
#pragma unroll
      for (int mw = 0; mw < TW; ++mw) {
        zz[mw] = zc[mw] + __shfl_xor(zc[mw], 32);
        if (!tv[mw]) continue;
        mzz = max(mzz, __builtin_bit_cast(u32, __builtin_fabsf(zz[mw])));
#pragma unroll
        for (int nt = 0; nt < DVT; ++nt)
#pragma unroll
          for (int r = 0; r < 16; ++r) ma = max(ma, __builtin_bit_cast(u32, __builtin_fabsf(acc[mw][nt][r])));
      }
      ma = wave_max_u32(ma);
      mzz = wave_max_u32(mzz);
      if (lane == 0) {
        red[0][w] = ma;
        red[2][w] = mzz;
      }
      __syncthreads();
      ma = red_max(0);
      mzz = red_max(2);
      const int ea = ma == 0u ? -1000 : (int)(ma >> 23) - 127 + eref;
      const int ez = mzz == 0u ? -1000 : (int)(mzz >> 23) - 127 + ezref;
      const int E = max(max(ea, ez) - 13, -100);
      // an all-zero part is stored as zeros (its scale could exceed fp32 when the other part
      // sets E, and 0 * inf would be NaN); a nonzero part's scale is at most 2^127, since
      // E >= its own exponent - 13 (values below 2^-114 of the slot's largest then flush)
      const float sc = ma == 0u ? 0.f : __builtin_ldexpf(1.0f, min(eref - E, 127));
      const float scz = mzz == 0u ? 0.f : __builtin_ldexpf(1.0f, min(ezref - E, 127));
      const size_t slot = (size_t)s * p.BH + bh;
      uint16_t* Ts = p.T + slot * (size_t)(FT::NGB * DVP * 64);
      uint16_t* Zs = p.Z + slot * (size_t)(FT::NGB * 64);
#pragma unroll
      for (int mw = 0; mw < TW; ++mw) {
        if (!tv[mw]) continue;
        const int tt = 8 * wga + TW * w + mw;
#pragma unroll
        for (int nt = 0; nt < DVT; ++nt) {
          const int row = 32 * nt + n;
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            const int f0 = 32 * tt + 8 * q4 + 4 * h;
            const int gb = f0 >> 6, uu = (f0 & 63) >> 3;
            const size_t off = (size_t)gb * (DVP * 64) + row * 64 + gswz(row, uu) + (f0 & 7);
            const f32x16& a = acc[mw][nt];
            *reinterpret_cast<u32x2*>(Ts + off) =
                (u32x2){pack_f16x2(a[4 * q4] * sc, a[4 * q4 + 1] * sc), pack_f16x2(a[4 * q4 + 2] * sc, a[4 * q4 + 3] * sc)};
          }
        }
        if (h == 0) Zs[32 * tt + n] = (uint16_t)(pack_f16x2(zz[mw] * scz, 0.f) & 0xffffu);
      }
      if (tid == 0) p.E[slot * nwga + wga] = E;
      // the stores out before the copy waits above count this wave's copies again
      wait_vm(0);
    }
  }
  if (TOTAL) {
    float* t = p.Tot + (((size_t)part * p.BH + bh) * nwga + wga) * (NT * PER) + tid * PER;
#pragma unroll
    for (int mw = 0; mw < TW; ++mw) {
#pragma unroll
      for (int nt = 0; nt < DVT; ++nt)
#pragma unroll
        for (int r = 0; r < 16; ++r) t[(mw * DVT + nt) * 16 + r] = acc[mw][nt][r];
      t[TW * DVT * 16 + mw] = zc[mw];
    }
  }
}

// ---------------------------------------------------------------- kernel 2: outputs
template <int DP, int DVT, bool VEC>
__global__ __launch_bounds__(256, DVT == 4 ? 1 : 2) void gout_kernel(const GParams p) {
  using FT = GFeat<DP>;
  constexpr int DB = DP / 16, DVP = 32 * DVT, KS = DP / 16;
  constexpr int NR = DP / 2 + 4;                 // rotated fp16 pairs of a'/m per token tile
  constexpr int NU = DP / 2 + 8;                 // unrotated pairs (a' through index DP + 15)
  constexpr int TB = DVP * 64 + 512;             // halves per T stage: block, then 1 KB of z
  constexpr int NS = 4;                          // T stages (blocks in flight: NS - 1)
  constexpr int NB = (FT::NG + 3) / 4;           // blocks holding groups the loop reads
  using Stager = BlockStager<KS, DVT, VEC, false>;
  constexpr int KROW = Stager::KROW;
  constexpr int IB = 2 * (BN * KROW + DVP * VROW);
  constexpr int BIG = NS * TB > IB ? NS * TB : IB;
  __shared__ __attribute__((aligned(16))) uint16_t Aq[(DP + 1) * GQ];
  __shared__ __attribute__((aligned(16))) uint16_t big[BIG];
  __shared__ float wtab[FT::NGP];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, n = lane & 31;
  const int N = p.N, d = p.d, dv = p.dv;
  const int ntile = (N + GQ - 1) / GQ;
  const int bh = blockIdx.x / ntile, tile = blockIdx.x - bh * ntile;
  const int t0 = tile * GQ, s = t0 / GL, seg0 = s * GL;
  const uint16_t* __restrict__ qg = p.q + (size_t)bh * N * d;
  const uint16_t* __restrict__ kg = p.k + (size_t)bh * N * d;
  const uint16_t* __restrict__ vg = p.v + (size_t)bh * N * dv;

  // ---- queries: raw bf16 fragments for the scores, a'/m as rotated fp16 pairs for the features
  u32x4 qf[2][KS];
  u32 R[2][NR];
  float m2[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int tok = t0 + 64 * w + 32 * nt + n;
    const bool ok = tok < N;
    u32 qp[DP / 2];
#pragma unroll
    for (int c = 0; c < DP / 8; ++c) {
      const u32x4 x = load_row8<VEC>(qg + (size_t)tok * d, 8 * c, d, ok);
#pragma unroll
      for (int e = 0; e < 4; ++e) qp[4 * c + e] = x[e];
    }
    // dims 16 kk + 8 h .. +7 (a bit select on the lane half: no array indexed by it)
    const u32 hm = 0u - (u32)h;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
#pragma unroll
      for (int e = 0; e < 4; ++e) qf[nt][kk][e] = (qp[8 * kk + e] & ~hm) | (qp[8 * kk + 4 + e] & hm);
    u32 mxb = 0u;
#pragma unroll
    for (int c = 0; c < DP / 2; ++c) {
      mxb = max(mxb, __builtin_bit_cast(u32, __builtin_fabsf(bf16_lo_to_f32(qp[c]) * p.scale)));
      mxb = max(mxb, __builtin_bit_cast(u32, __builtin_fabsf(bf16_hi_to_f32(qp[c]) * p.scale)));
    }
    // m = 2^e >= max(max |a|, 1): a'/m in [-1, 1]
    const float mxf = __builtin_fmaxf(__builtin_bit_cast(float, mxb), 1.0f);
    int e;
    (void)__builtin_frexpf(mxf, &e);
    const float inv = __builtin_ldexpf(1.0f, -e);
    m2[nt] = __builtin_ldexpf(1.0f, 2 * e);
    u32 U[NU];
#pragma unroll
    for (int c = 0; c < NU; ++c) {
      if (c < DP / 2)
        U[c] = pack_f16x2(bf16_lo_to_f32(qp[c]) * p.scale * inv, bf16_hi_to_f32(qp[c]) * p.scale * inv);
      else if (c == DP / 2)
        U[c] = pack_f16x2(inv, 0.f);
      else
        U[c] = 0u;
    }
    // lane half 1 takes the pairs four further on
#pragma unroll
    for (int c = 0; c < NR; ++c) R[nt][c] = (U[c] & ~hm) | (U[c + 4] & hm);
    if (h == 0) {
      const int tl = 64 * w + 32 * nt + n;
#pragma unroll
      for (int c = 0; c <= DP / 2; ++c) {
        Aq[(2 * c) * GQ + tl] = (uint16_t)(U[c] & 0xffffu);
        if (2 * c + 1 <= DP) Aq[(2 * c + 1) * GQ + tl] = (uint16_t)(U[c] >> 16);
      }
    }
  }

  f32x16 acc[DVT][2];
  float den[2] = {0.f, 0.f};
#pragma unroll
  for (int mt = 0; mt < DVT; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = splat16(0.f);

  // ---- the earlier segments, through the prefix state of segment s
  if (s >= 1) {
    const size_t slot = (size_t)(s - 1) * p.BH + bh;
    const int* Es = p.E + slot * FT::NWGA;
    int emax = -1000;
#pragma unroll
    for (int x = 0; x < FT::NWGA; ++x) emax = max(emax, Es[x]);
    for (int g = tid; g < FT::NGP; g += 256)
      wtab[g] = group_weight<DP>(g) * __builtin_ldexpf(1.0f, Es[g >> 4] - emax);
    const u32x4 rT = buffer_rsrc(p.T + slot * (size_t)(FT::NGB * DVP * 64), (u32)(FT::NGB * DVP * 128));
    const u32x4 rZ = buffer_rsrc(p.Z + slot * (size_t)(FT::NGB * 64), (u32)(FT::NGB * 128));
    constexpr int UT = DVP / 8;   // 1 KB units of a T block, then one of z
    const int my_units = (UT + 1) / 4 + (w < (UT + 1) % 4 ? 1 : 0);
    auto issue = [&](int gb) {
      if (gb >= NB) return;
      const u32 base = lds_addr(&big[(gb % NS) * TB]);
      for (int u = w; u <= UT; u += 4) {
        if (u < UT)
          lds_copy16(rT, base + 1024 * u, gb * (DVP * 128) + 1024 * u + 16 * lane);
        else
          lds_copy16(rZ, base + DVP * 128, gb * 128 + 16 * lane);
      }
    };
    for (int b = 0; b < NS - 1; ++b) issue(b);
    int g = 0;
    for (int i = 0; i <= DP; ++i) {
      float ai[2];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
        ai[nt] = (float)__builtin_bit_cast(_Float16, Aq[i * GQ + 64 * w + 32 * nt + n]);
      const int js = i < DP ? (i >> 4) : 0, je = i < DP ? DB - 1 : DB;
#pragma unroll
      for (int J = 0; J <= DB; ++J) {
        if (J < js || J > je) continue;
        if ((g & 3) == 0) {
          // this wave's copies of block g / 4 landed, then every wave's; every wave is also done
          // with the block before, whose stage the next copy reuses
          const int b = g >> 2;
          wait_vm(my_units * min(NS - 2, NB - 1 - b));
          __syncthreads();
          issue(b + NS - 1);
        }
        const uint16_t* st = &big[((g >> 2) % NS) * TB];
        const int sl = g & 3;
        const float wg = wtab[g];
        u32x4 tf[DVT];
#pragma unroll
        for (int mt = 0; mt < DVT; ++mt) {
          const int row = 32 * mt + n;
          tf[mt] = *reinterpret_cast<const u32x4*>(st + row * 64 + gswz(row, 2 * sl + h));
        }
        const u32x4 zr = *reinterpret_cast<const u32x4*>(st + DVP * 64 + 16 * sl + 8 * h);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          const float a = ai[nt] * wg;
          const u32 ap = pack_f16x2(a, a);
          const u32x4 bf = {pk_mul_f16(ap, R[nt][8 * J]), pk_mul_f16(ap, R[nt][8 * J + 1]),
                            pk_mul_f16(ap, R[nt][8 * J + 2]), pk_mul_f16(ap, R[nt][8 * J + 3])};
#pragma unroll
          for (int c = 0; c < 4; ++c) den[nt] = dot2_f16(bf[c], zr[c], den[nt]);
#pragma unroll
          for (int mt = 0; mt < DVT; ++mt) acc[mt][nt] = mfma32x32x16_f16(tf[mt], bf, acc[mt][nt]);
        }
        ++g;
      }
    }
    __syncthreads();   // every wave done with the T stages before the key blocks reuse them
    const int eh = head_vexp(p, bh);   // the prefixes hold V / 2^Eh
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      den[nt] *= __builtin_ldexpf(m2[nt], emax);
      const float f = __builtin_ldexpf(m2[nt], emax + eh);
#pragma unroll
      for (int mt = 0; mt < DVT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[mt][nt][r] *= f;
    }
  }

  // ---- keys of this segment up to the queries: p = 1 + s + s^2/2 directly
  // key blocks: K [2][BN][KROW], then V^T [2][DVP][VROW]
  auto kbuf = [&](int b) -> uint16_t* { return big + b * (BN * KROW); };
  auto vbuf = [&](int b) -> uint16_t* { return big + 2 * BN * KROW + b * (DVP * VROW); };
  const int kend = min(t0 + GQ, N);
  const int nblk = (kend - seg0 + BN - 1) / BN;
  const int wlast = min(t0 + 64 * w + 63, N - 1);
  Stager stg;
  stg.load(kg, vg, seg0, N, d, dv, tid);
  stg.store(kbuf(0), vbuf(0), tid);
  __syncthreads();
  for (int j = 0; j < nblk; ++j) {
    const int kb = seg0 + BN * j;
    const bool more = j + 1 < nblk;
    if (more) stg.load(kg, vg, kb + BN, N, d, dv, tid);
    const uint16_t* kt = kbuf(j & 1);
    const uint16_t* vt = vbuf(j & 1);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int kb2 = kb + 32 * ks;
      if (kb2 > wlast) break;
      u32x4 kf[KS];
#pragma unroll
      for (int kk = 0; kk < KS; ++kk)
        kf[kk] = *reinterpret_cast<const u32x4*>(kt + (32 * ks + n) * KROW + 16 * kk + 8 * h);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int tb = t0 + 64 * w + 32 * nt;
        if (kb2 > tb + 31 || tb >= N) continue;
        f32x16 sc = splat16(0.f);
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) sc = mfma32x32x16(kf[kk], qf[nt][kk], sc);
        const int tok = tb + n;
        float pv[16];
        // tiles wholly below the diagonal and inside the sequence need no mask
        const bool masked = kb2 + 31 > tb || kb2 + 31 >= N;
        if (masked) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float x = sc[r] * p.scale;
            const int key = kb2 + c32_row(r, h);
            pv[r] = (key > tok || key >= N) ? 0.f : __builtin_fmaf(x, __builtin_fmaf(0.5f, x, 1.0f), 1.0f);
          }
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float x = sc[r] * p.scale;
            pv[r] = __builtin_fmaf(x, __builtin_fmaf(0.5f, x, 1.0f), 1.0f);
          }
        }
        // p as bf16 hi + lo (16 significant bits; V is exact in bf16), and the row sums from the
        // same two parts, so that the rounding of a row cancels in the quotient
        u32x4 pf[2], pl[2];
#pragma unroll
        for (int m = 0; m < 2; ++m) {
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const float x0 = pv[8 * m + 2 * c], x1 = pv[8 * m + 2 * c + 1];
            const u32 hi = pack_bf16x2(x0, x1);
            const u32 lo = pack_bf16x2(x0 - bf16_lo_to_f32(hi), x1 - bf16_hi_to_f32(hi));
            pf[m][c] = hi;
            pl[m][c] = lo;
            den[nt] = dot2_bf16(lo, kOnesBf16, dot2_bf16(hi, kOnesBf16, den[nt]));
          }
        }
#pragma unroll
        for (int mt = 0; mt < DVT; ++mt)
#pragma unroll
          for (int m = 0; m < 2; ++m) {
            const uint16_t* vp = vt + (32 * mt + n) * VROW + 32 * ks + 16 * m + 4 * h;
            const u32x2 a0 = *reinterpret_cast<const u32x2*>(vp);
            const u32x2 a1 = *reinterpret_cast<const u32x2*>(vp + 8);
            const u32x4 vf = {a0[0], a0[1], a1[0], a1[1]};
            acc[mt][nt] = mfma32x32x16(vf, pf[m], acc[mt][nt]);
            acc[mt][nt] = mfma32x32x16(vf, pl[m], acc[mt][nt]);
          }
      }
    }
    if (more) stg.store(kbuf((j + 1) & 1), vbuf((j + 1) & 1), tid);
    __syncthreads();
  }

  // ---- out = num / (den + eps)
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    float dd = den[nt];
    dd += __shfl_xor(dd, 32);
    const float inv = p.normalize ? 1.0f / (dd + p.eps) : 1.0f;
    const int tok = t0 + 64 * w + 32 * nt + n;
    if (tok >= N) continue;
    if (h == 0 && p.den_out != nullptr) p.den_out[(size_t)bh * N + tok] = dd;
    const size_t ob = ((size_t)bh * N + tok) * dv;
#pragma unroll
    for (int mt = 0; mt < DVT; ++mt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const float y[4] = {acc[mt][nt][4 * q4] * inv, acc[mt][nt][4 * q4 + 1] * inv, acc[mt][nt][4 * q4 + 2] * inv,
                            acc[mt][nt][4 * q4 + 3] * inv};
        store_out4<VEC>(p.out, p.out_f32 != 0, ob, 32 * mt + 8 * q4 + 4 * h, dv, y);
      }
  }
}

int dp_of(int d) { return 16 * ((d + 15) / 16); }
int dvt_of(int dv) { return dv <= 32 ? 1 : dv <= 64 ? 2 : 4; }

// Parts of the state sweep: when the (head, work-group) pairs fill less than half of 256 CUs,
// enough parts for two work-groups per CU (the totals pass sweeps all but the last part a second
// time, which pays only then), at least two segments per part.
void state_parts(int BH, int nwga, int nseg, int& nparts, int& spp) {
  const int units = BH * nwga;
  const int want = units < 128 ? (512 + units - 1) / units : 1;
  nparts = max(1, min(want, (nseg - 1) / 2));
  spp = (nseg - 1 + nparts - 1) / nparts;
  nparts = (nseg - 1 + spp - 1) / spp;
}

// Workspace regions of one call: per (segment slot, head) the T blocks, z and the exponents; per
// (head, chunk before the last segment) the converted chunk and its two exponents; the part
// totals of the state sweep.
struct GLayout {
  size_t t, z, e, kv, ce, tot, vm, total;
  int nparts, spp;
};

template <int DP>
GLayout glayout_dp(int BH, int nseg, int DVT) {
  using FT = GFeat<DP>;
  const size_t nslot = (size_t)(nseg - 1) * BH;
  const size_t nchk = (size_t)(nseg - 1) * (GL / GC) * BH;
  size_t halves = 0;
  switch (DVT) {
    case 1: halves = GChunk<DP, 1>::HALVES; break;
    case 2: halves = GChunk<DP, 2>::HALVES; break;
    default: halves = GChunk<DP, 4>::HALVES; break;
  }
  const auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
  GLayout L{};
  L.t = 0;
  L.z = L.t + up(nslot * FT::NGB * 64 * (32 * DVT) * 2);
  L.e = L.z + up(nslot * FT::NGB * 64 * 2);
  L.kv = L.e + up(nslot * FT::NWGA * 4);
  L.ce = L.kv + up(nchk * halves * 2);
  L.tot = L.ce + up(nchk * 8);
  state_parts(BH, FT::NWGA, nseg, L.nparts, L.spp);
  // per state work-group of every part but the last: its eight tiles' sums, 32 x DVT accumulators
  // and a z partial per lane
  L.vm = L.tot + up((size_t)(L.nparts - 1) * BH * FT::NWGA * 512 * (DVT * 16 + 1) * 4);
  L.total = L.vm + up((size_t)BH * kVmParts * 4);
  return L;
}

GLayout glayout(int BH, int N, int d, int dv) {
  const int nseg = (N + GL - 1) / GL, DP = dp_of(d), DVT = dvt_of(dv);
  switch (DP) {
    case 16: return glayout_dp<16>(BH, nseg, DVT);
    case 32: return glayout_dp<32>(BH, nseg, DVT);
    case 48: return glayout_dp<48>(BH, nseg, DVT);
    default: return glayout_dp<64>(BH, nseg, DVT);
  }
}

// 32-feature tiles per wave of the state kernel: one (8 waves of at most 128 VGPRs, two
// work-groups per CU) up to dv = 64; two (4 waves) for dv = 128, whose accumulators need more
template <int DVT>
constexpr int state_tw() { return DVT == 4 ? 2 : 1; }

template <int DP, int DVT>
int launch_g(const GParams& p, hipStream_t stream) {
  using FT = GFeat<DP>;
  if (p.nseg > 1) {
    const int nch = (p.nseg - 1) * (GL / GC);
    hipLaunchKernelGGL(gvmax_kernel, dim3((unsigned)kVmParts, (unsigned)p.BH), dim3(256), 0, stream, p);
    int e = (int)hipGetLastError();
    if (e != 0) return e;
    hipLaunchKernelGGL((gprep_kernel<DP, DVT>), dim3((unsigned)(p.BH * nch)), dim3(256), 0, stream, p);
    e = (int)hipGetLastError();
    if (e != 0) return e;
    const unsigned units = (unsigned)(p.BH * FT::NWGA);
    const long long cus = device_cu_count();
    GParams ps = p;
    if (p.nparts > 1) {
      ps.alt_prio = (long long)units * (p.nparts - 1) > cus ? 1 : 0;
      hipLaunchKernelGGL((gstate_kernel<DP, DVT, true, state_tw<DVT>()>), dim3(units * (unsigned)(p.nparts - 1)),
                         dim3(64 * (8 / state_tw<DVT>())), 0, stream, ps);
      e = (int)hipGetLastError();
      if (e != 0) return e;
    }
    ps.alt_prio = (long long)units * p.nparts > cus ? 1 : 0;
    hipLaunchKernelGGL((gstate_kernel<DP, DVT, false, state_tw<DVT>()>), dim3(units * (unsigned)p.nparts),
                       dim3(64 * (8 / state_tw<DVT>())), 0, stream, ps);
    e = (int)hipGetLastError();
    if (e != 0) return e;
  }
  const dim3 grid((unsigned)(p.BH * ((p.N + GQ - 1) / GQ)));
  if (p.vec)
    hipLaunchKernelGGL((gout_kernel<DP, DVT, true>), grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((gout_kernel<DP, DVT, false>), grid, dim3(256), 0, stream, p);
  return (int)hipGetLastError();
}

template <int DP>
int launch_dp(const GParams& p, int DVT, hipStream_t stream) {
  switch (DVT) {
    case 1: return launch_g<DP, 1>(p, stream);
    case 2: return launch_g<DP, 2>(p, stream);
    default: return launch_g<DP, 4>(p, stream);
  }
}

}  // namespace

bool general_chunked_shape(int d, int dv, bool in_f32) {
  (void)in_f32;
  return d >= 1 && d <= 64 && dv >= 1 && dv <= 128;
}

size_t general_chunked_bytes(int BH, int N, int d, int dv, bool in_f32) {
  if (!general_chunked_shape(d, dv, in_f32)) return (size_t)-1;
  if (in_f32) return general_chunked_f32_bytes(BH, N, d, dv);
  const int nseg = (N + GL - 1) / GL;
  if (nseg <= 1) return 0;
  return glayout(BH, N, d, dv).total;
}

int launch_general_chunked(const ChunkedArgs& a, hipStream_t stream) {
  if (!general_chunked_shape(a.d, a.dv, a.in_f32)) return LA_ERR_UNSUPPORTED_DIM;
  if (a.in_f32) return launch_general_chunked_f32(a, stream);
  const int DP = dp_of(a.d), DVT = dvt_of(a.dv);
  GParams p{};
  p.q = static_cast<const uint16_t*>(a.q);
  p.k = static_cast<const uint16_t*>(a.k);
  p.v = static_cast<const uint16_t*>(a.v);
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
  const auto al = [](const void* x, int b) { return (reinterpret_cast<uintptr_t>(x) & (uintptr_t)(b - 1)) == 0; };
  // vector paths: 16-byte rows of q, k (d % 8), 8-byte rows of v and the output (dv % 4)
  p.vec = (a.d % 8 == 0 && a.dv % 4 == 0 && al(a.q, 16) && al(a.k, 16) && al(a.v, 16) &&
           al(a.out, 16))
              ? 1
              : 0;
  if (p.nseg > 1) {
    const size_t need = general_chunked_bytes(a.BH, a.N, a.d, a.dv, a.in_f32);
    if (a.workspace == nullptr || a.workspace_bytes < need) return LA_ERR_WORKSPACE;
    if (!al(a.workspace, 16)) return LA_ERR_BAD_ALIGNMENT;
    const GLayout L = glayout(a.BH, a.N, a.d, a.dv);
    char* ws = static_cast<char*>(a.workspace);
    p.T = reinterpret_cast<uint16_t*>(ws + L.t);
    p.Z = reinterpret_cast<uint16_t*>(ws + L.z);
    p.E = reinterpret_cast<int*>(ws + L.e);
    p.KV = reinterpret_cast<uint16_t*>(ws + L.kv);
    p.CE = reinterpret_cast<u32x2*>(ws + L.ce);
    p.Tot = reinterpret_cast<float*>(ws + L.tot);
    p.VM = reinterpret_cast<u32*>(ws + L.vm);
    p.nparts = L.nparts;
    p.spp = L.spp;
  }
  switch (DP) {
    case 16: return launch_dp<16>(p, DVT, stream);
    case 32: return launch_dp<32>(p, DVT, stream);
    case 48: return launch_dp<48>(p, DVT, stream);
    default: return launch_dp<64>(p, DVT, stream);
  }
}

}  // namespace la
