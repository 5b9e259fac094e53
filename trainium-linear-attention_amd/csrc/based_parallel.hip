// Fused causal BASED attention, parallel (quadratic) form, for gfx950.
//
// Replaces the NKI parallel kernel (kernels/nki_attention.py:33-115) and the host-side
// normalisation of solution_nki (kernels/pytorch_attention.py:44-78).
//
// Math.  With a = q.k (unscaled), c = scale and s = c a:
//     p = 1 + s + s^2/2 = 1 + (c^2/2) u,   u = a^2 + 2a/c = (a + 1/c)^2 - 1/c^2.
// The score MFMA is started from an accumulator filled with 1/c, so it produces b = a + 1/c
// and u costs one FMA (b*b - 1/c^2).  This is phi(q).phi(k) of the Taylor feature map
// (benchmarks/chunked_attention_benchmark.py:34-53) evaluated through the exact identity
// phi(q).phi(k) = 1 + s + s^2/2, so phi is never materialised.
//
// Precision.  The P.V product runs as an fp16 MFMA: V is converted bf16 -> fp16 while it is
// staged (exact for 2^-14 <= |v| <= 65504) and u is rounded to fp16 (2^-11 relative, 8x finer
// than bf16).  Q is pre-scaled by 2^-k (exact) so that the rounded quantity is u * 2^-2k ~ r
// and stays far from fp16 overflow (|q.k| * scale < ~255).  The constant 1 of p is kept exact:
//   * key blocks strictly before the work-group's queries contribute sum(v) through an fp32
//     running column sum of V (v_dot2 against packed ones), snapshotted per wave;
//   * the wave's own diagonal block adds its causal "ones" through a second MFMA whose B
//     operand is the causal mask times the weight of "1" in u units (split hi + lo in fp16;
//     exact for scale = 1/sqrt(d)).
// Then num = acc / W + vsum and den = (t + 1) + rowsum(fp16(u)) / W, the row sum taken over the
// same rounded u that feeds the MFMA.
//
// Tiling.  4 waves per work-group; each wave owns 32*QT queries (QT 32x32 N-tiles) and the
// full dv (MT 32-row M-tiles of the transposed output O^T = V^T P^T).  Keys stream through LDS
// in blocks of 64 (double buffered): K row-major [key][d], V transposed [dv][key] so both
// MFMA operands are contiguous 8-byte / 16-byte LDS reads.  Scores are computed transposed,
// S^T = K Q^T, so the score accumulator layout is directly the B operand layout of the PV
// MFMA (no cross-lane shuffles).
#include "la_common.hpp"
#include "la_internal.hpp"
#include "la_stage.hpp"

namespace la {

namespace {

struct ParallelParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  void* out;
  float* den;
  int BH, N, d, dv, nqb;
  float inv_c, inv_c2, fscale, eps;
  float qscale;           // 2^-k applied to q (exact in bf16)
  u32 ones_hi, ones_lo;   // fp16 bits of the weight W of "1" in u units, hi + lo (both halves)
  int normalize, out_f32;
};

// UNIT: 1/c scales to exactly 1 (scale = 1/sqrt(d) with d a power of 4), so the score MFMA
// starts from the inline constant 1.0 and u = b*b - 1.
//
// DMA (d = 16, dv % 8 == 0): K and V blocks are copied global -> LDS by buffer_load ... lds
// (no staging registers, out-of-range rows read as zero) three blocks ahead into four raw
// stages; V is converted to fp16 and transposed LDS -> LDS one block ahead.  Barriers are
// plain s_barrier with explicit vmcnt / lgkmcnt waits so that in-flight copies are not drained.
template <int KS, int MT, int QT, bool VEC, bool UNIT, bool DMA, class KsT, class VTsT, class SnapT, class KrawT,
          class VrawT>
__device__ __forceinline__ void based_parallel_body(const ParallelParams& p, KsT* __restrict__ Ks,
                                                    VTsT* __restrict__ VTs, SnapT* __restrict__ snap,
                                                    KrawT* __restrict__ Kraw, VrawT* __restrict__ Vraw) {
  constexpr int DK = 16 * KS, DV = 32 * MT, BM = 128 * QT, NSNAP = BM / BN;
  constexpr int KROW = DK + 8;
  constexpr int LPR = 256 / DV;      // threads per V^T row in the running column sum
  constexpr int KPL = BN / LPR;      // keys per thread in the running column sum
  using Stager = BlockStager<KS, MT, VEC, true>;
  static_assert(!DMA || KS == 1, "DMA staging is for d = 16");
  constexpr int NRAW = 4;                 // raw DMA stages
  constexpr int NKU = 2, NVU = DV / 8;    // 1 KB DMA units per block (K, V)
  constexpr int NU = NKU + NVU;

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, h = lane >> 5, n = lane & 31;
  const int N = p.N, d = p.d, dv = p.dv;

  int bh, qb;
  map_causal_block(blockIdx.x, p.BH, p.nqb, bh, qb);
  const int q0 = qb * BM;
  const int jb0 = q0 / BN;
  const int nblk = min((N + BN - 1) / BN, (q0 + BM) / BN);
  const size_t hrow = (size_t)bh * N;
  const uint16_t* __restrict__ qg = p.q + hrow * d;
  const uint16_t* __restrict__ kg = p.k + hrow * d;
  const uint16_t* __restrict__ vg = p.v + hrow * dv;

  const int wq0 = q0 + 32 * QT * w;    // first query of this wave
  const int jd = wq0 / BN;             // this wave's diagonal key block
  const bool wave_live = wq0 < N;

  // Q fragments (B operand of S^T = K Q^T): lane holds q[query][16kk + 8h .. +7].
  u32x4 qf[QT][KS];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int query = wq0 + 32 * qt + n;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const int col = 16 * kk + 8 * h;
      u32x4 x = {0u, 0u, 0u, 0u};
      if (query < N) {
        const uint16_t* src = qg + (size_t)query * d + col;
        if (VEC) {
          if (col < d) x = *reinterpret_cast<const u32x4*>(src);
        } else {
          uint16_t e[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) e[i] = (col + i < d) ? src[i] : (uint16_t)0;
          x = (u32x4){e[0] | ((u32)e[1] << 16), e[2] | ((u32)e[3] << 16), e[4] | ((u32)e[5] << 16),
                      e[6] | ((u32)e[7] << 16)};
        }
      }
      qf[qt][kk] = scale_bf16x8(x, p.qscale);
    }
  }

  f32x16 acc[QT][MT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[qt][mt] = splat16(0.f);
  float rsum[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) rsum[qt] = 0.f;

  // running column sum of V over blocks [0, jb0 + s) for snapshot s: thread -> (row, segment)
  const int vs_row = tid / LPR, vs_seg = tid % LPR;
  float vacc = 0.f;
  constexpr u32 kOnes = 0x3c003c00u;  // packed fp16 (1, 1)

  const float inv_c = UNIT ? 1.0f : p.inv_c, inv_c2 = UNIT ? 1.0f : p.inv_c2;

  // ---- DMA staging helpers
  const int wu = __builtin_amdgcn_readfirstlane(w);
  const int my_units = NU / 4 + (wu < NU % 4 ? 1 : 0);
  const u32x4 rk = buffer_rsrc(kg, (u32)N * 32u);
  const u32x4 rv = buffer_rsrc(vg, (u32)N * (u32)dv * 2u);
  auto issue_dma = [&](int blk) {
    const int st = blk & (NRAW - 1);
    const int row0 = blk * BN;
#pragma unroll
    for (int i = 0; i < (NU + 3) / 4; ++i) {
      const int u = wu + 4 * i;
      if (u >= NU) break;
      if (u < NKU) {
        // K slot sl = 2 key + (c ^ ((key >> 2) & 1)): 16-byte chunk c of key row, swizzled
        const int sl = 64 * u + lane, key = sl >> 1, c = (sl & 1) ^ ((key >> 2) & 1);
        lds_copy16(rk, lds_addr(&Kraw[st][512 * u]), ((row0 + key) * 16 + 8 * c) * 2);
      } else {
        const int ch = 64 * (u - NKU) + lane, key = ch / (DV / 8), col = 8 * (ch % (DV / 8));
        const int off = col < dv ? ((row0 + key) * dv + col) * 2 : 0x7ffffff0;
        lds_copy16(rv, lds_addr(&Vraw[st][512 * (u - NKU)]), off);
      }
    }
  };
  // raw V of block blk (bf16 [key][DV]) -> VTs[blk & 1] (fp16 [dv][key])
  auto convert_v = [&](int blk) {
    const uint16_t* src = &Vraw[blk & (NRAW - 1)][0];
    uint16_t* dstb = &VTs[blk & 1][0];
#pragma unroll
    for (int g = tid; g < (DV / 4) * (BN / 4); g += 256) {
      const int g4 = g % (DV / 4), kg4 = g / (DV / 4);
      u32x2 x[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = *reinterpret_cast<const u32x2*>(&src[(4 * kg4 + i) * DV + 4 * g4]);
      const u32 a0 = x[0][0], a1 = x[1][0], a2 = x[2][0], a3 = x[3][0];
      const u32 b0 = x[0][1], b1 = x[1][1], b2 = x[2][1], b3 = x[3][1];
      uint16_t* dst = dstb + (4 * g4) * VROW + 4 * kg4;
      *reinterpret_cast<u32x2*>(dst) = (u32x2){pack_f16x2(bf16_lo_to_f32(a0), bf16_lo_to_f32(a1)),
                                               pack_f16x2(bf16_lo_to_f32(a2), bf16_lo_to_f32(a3))};
      *reinterpret_cast<u32x2*>(dst + VROW) = (u32x2){pack_f16x2(bf16_hi_to_f32(a0), bf16_hi_to_f32(a1)),
                                                      pack_f16x2(bf16_hi_to_f32(a2), bf16_hi_to_f32(a3))};
      *reinterpret_cast<u32x2*>(dst + 2 * VROW) = (u32x2){pack_f16x2(bf16_lo_to_f32(b0), bf16_lo_to_f32(b1)),
                                                          pack_f16x2(bf16_lo_to_f32(b2), bf16_lo_to_f32(b3))};
      *reinterpret_cast<u32x2*>(dst + 3 * VROW) = (u32x2){pack_f16x2(bf16_hi_to_f32(b0), bf16_hi_to_f32(b1)),
                                                          pack_f16x2(bf16_hi_to_f32(b2), bf16_hi_to_f32(b3))};
    }
  };
  // LDS-only barrier: my LDS writes done, then s_barrier; the asm clobbers keep the compiler
  // from moving memory operations across it.
  auto lds_barrier = [&]() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0), vmcnt/expcnt unchanged
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // wait until at most `left` DMA units of this wave are still in flight
  auto wait_dma = [&](int left) {
    asm volatile("" ::: "memory");
    if (left >= 6) __builtin_amdgcn_s_waitcnt(0x0f76);
    else if (left == 5) __builtin_amdgcn_s_waitcnt(0x0f75);
    else if (left == 4) __builtin_amdgcn_s_waitcnt(0x0f74);
    else if (left == 3) __builtin_amdgcn_s_waitcnt(0x0f73);
    else if (left == 2) __builtin_amdgcn_s_waitcnt(0x0f72);
    else if (left == 1) __builtin_amdgcn_s_waitcnt(0x0f71);
    else __builtin_amdgcn_s_waitcnt(0x0f70);
    asm volatile("" ::: "memory");
  };
  auto kfrag = [&](int j, int ks, int kk) -> u32x4 {
    if (DMA) {
      const int key = 32 * ks + n;
      const int sl = 2 * key + (h ^ ((key >> 2) & 1));
      return *reinterpret_cast<const u32x4*>(&Kraw[j & (NRAW - 1)][8 * sl]);
    }
    return *reinterpret_cast<const u32x4*>(&Ks[j & 1][(32 * ks + n) * KROW + 16 * kk + 8 * h]);
  };

  Stager st;
  if (DMA) {
    // drain the Q loads so only DMA units are counted by vmcnt from here on
    __builtin_amdgcn_s_waitcnt(0x0f70);
    issue_dma(0);
    if (nblk > 1) issue_dma(1);
    if (nblk > 2) issue_dma(2);
    wait_dma(my_units * ((nblk > 2) ? 2 : (nblk > 1 ? 1 : 0)));
    lds_barrier();
    convert_v(0);
    if (jb0 == 0) snap[0][tid] = 0.f;
  } else {
    st.load(kg, vg, 0, N, d, dv, tid);
    st.store(Ks[0], VTs[0], tid);
    if (jb0 == 0) snap[0][tid] = 0.f;
    __syncthreads();
  }

  for (int j = 0; j < nblk; ++j) {
    const int s = j & 1;
    if (DMA) {
      // block j+1 must have landed; blocks j+2 (and j+3 once issued) may still be in flight
      wait_dma(j + 2 < nblk ? my_units : 0);
      lds_barrier();
      if (j + 3 < nblk) issue_dma(j + 3);
      if (j + 1 < nblk) convert_v(j + 1);
    } else {
      if (j + 1 < nblk) st.load(kg, vg, (j + 1) * BN, N, d, dv, tid);
    }

    if (j <= jb0 + NSNAP - 2) {
      const uint16_t* src = &VTs[s][vs_row * VROW + vs_seg * KPL];
#pragma unroll
      for (int e = 0; e < KPL; e += 4) {
        const u32x2 x = *reinterpret_cast<const u32x2*>(src + e);
        vacc = dot2_f16(x[0], kOnes, vacc);
        vacc = dot2_f16(x[1], kOnes, vacc);
      }
      const int si = j - jb0 + 1;
      if (si >= 0 && si < NSNAP) snap[si][tid] = vacc;
    }

    if (wave_live && j < jd) {
      // Full block: every key precedes every query of this wave -- no mask, no "1" term
      // (the running column sum covers it).  All score MFMAs first, then the P.V MFMAs.
      u32x4 pf[2][QT][2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        u32x4 kf[KS];
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) kf[kk] = kfrag(j, ks, kk);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          f32x16 b = splat16(inv_c);
#pragma unroll
          for (int kk = 0; kk < KS; ++kk) b = mfma32x32x16(kf[kk], qf[qt][kk], b);
          float r = rsum[qt];
#pragma unroll
          for (int m = 0; m < 2; ++m) {
            u32 w[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              const int i = 8 * m + 2 * c;
              w[c] = pack_f16x2(__builtin_fmaf(b[i], b[i], -inv_c2), __builtin_fmaf(b[i + 1], b[i + 1], -inv_c2));
              r = dot2_f16(w[c], kOnes, r);
            }
            pf[ks][qt][m] = (u32x4){w[0], w[1], w[2], w[3]};
          }
          rsum[qt] = r;
        }
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int m = 0; m < 2; ++m) {
            const uint16_t* vp = &VTs[s][(32 * mt + n) * VROW + 32 * ks + 16 * m + 4 * h];
            const u32x2 a0 = *reinterpret_cast<const u32x2*>(vp);
            const u32x2 a1 = *reinterpret_cast<const u32x2*>(vp + 8);
            const u32x4 vf = {a0[0], a0[1], a1[0], a1[1]};
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) acc[qt][mt] = mfma32x32x16_f16(vf, pf[ks][qt][m], acc[qt][mt]);
          }
    } else if (wave_live && j == jd) {
      // Diagonal block: causal mask on u, plus the exact "1" of p through a mask MFMA.
      constexpr bool diag_block = true;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int kb = j * BN + 32 * ks;
        if (kb > wq0 + 32 * QT - 1) break;
        u32x4 kf[KS];
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) kf[kk] = kfrag(j, ks, kk);

        u32x4 pf[QT][2];
        u32x4 mk[QT][2];
        bool act[QT];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const int qbase = wq0 + 32 * qt;
          act[qt] = (kb <= qbase + 31) && (qbase < N);
          if (!act[qt]) continue;
          f32x16 b = splat16(inv_c);
#pragma unroll
          for (int kk = 0; kk < KS; ++kk) b = mfma32x32x16(kf[kk], qf[qt][kk], b);
          float u[16];
#pragma unroll
          for (int i = 0; i < 16; ++i) u[i] = __builtin_fmaf(b[i], b[i], -inv_c2);
          const int query = qbase + n;
          if (kb + 31 > qbase) {
#pragma unroll
            for (int i = 0; i < 16; ++i)
              if (kb + c32_row(i, h) > query) u[i] = 0.f;
          }
#pragma unroll
          for (int m = 0; m < 2; ++m) {
            pf[qt][m] = (u32x4){pack_f16x2(u[8 * m + 0], u[8 * m + 1]), pack_f16x2(u[8 * m + 2], u[8 * m + 3]),
                                pack_f16x2(u[8 * m + 4], u[8 * m + 5]), pack_f16x2(u[8 * m + 6], u[8 * m + 7])};
            float r = rsum[qt];
            r = dot2_f16(pf[qt][m][0], kOnes, r);
            r = dot2_f16(pf[qt][m][1], kOnes, r);
            r = dot2_f16(pf[qt][m][2], kOnes, r);
            r = dot2_f16(pf[qt][m][3], kOnes, r);
            rsum[qt] = r;
          }
          if (diag_block) {
            // causal mask times W for the exact "1" of p; element e <-> key
            // kb + 16m + 8(e/4) + 4h + (e%4)
#pragma unroll
            for (int m = 0; m < 2; ++m) {
              u32 wd[4];
#pragma unroll
              for (int e2 = 0; e2 < 4; ++e2) {
                const int e = 2 * e2;
                const int key0 = kb + 16 * m + 8 * (e >> 2) + 4 * h + (e & 3);
                const u32 lo = (key0 <= query) ? (p.ones_hi & 0xffffu) : 0u;
                const u32 hi = (key0 + 1 <= query) ? (p.ones_hi & 0xffff0000u) : 0u;
                wd[e2] = lo | hi;
              }
              mk[qt][m] = (u32x4){wd[0], wd[1], wd[2], wd[3]};
            }
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
              acc[qt][mt] = mfma32x32x16_f16(vf, pf[qt][m], acc[qt][mt]);
              if (diag_block) {
                acc[qt][mt] = mfma32x32x16_f16(vf, mk[qt][m], acc[qt][mt]);
                if (p.ones_lo != 0u) {
                  // same mask pattern, low part of 2/c^2
                  u32x4 ml;
#pragma unroll
                  for (int t = 0; t < 4; ++t) {
                    const u32 wv = mk[qt][m][t];
                    ml[t] = ((wv & 0xffffu) ? (p.ones_lo & 0xffffu) : 0u) |
                            ((wv & 0xffff0000u) ? (p.ones_lo & 0xffff0000u) : 0u);
                  }
                  acc[qt][mt] = mfma32x32x16_f16(vf, ml, acc[qt][mt]);
                }
              }
            }
          }
        }
      }
    }

    if (!DMA) {
      if (j + 1 < nblk) st.store(Ks[s ^ 1], VTs[s ^ 1], tid);
      __syncthreads();
    }
  }
  if (DMA) lds_barrier();   // snapshots written in the last iterations

  if (!wave_live) return;

  // epilogue: num = acc/W + vsum, den = (t+1) + rowsum/W  (fscale = 1/W)
  const int si = jd - jb0;
  float vsum[MT][16];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = 32 * mt + c32_row(i, h);
      float t = 0.f;
#pragma unroll
      for (int sg = 0; sg < LPR; ++sg) t += snap[si][row * LPR + sg];
      vsum[mt][i] = t;
    }

  const float fscale = p.fscale;
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const float rs = rsum[qt] + __shfl_xor(rsum[qt], 32);
    const int query = wq0 + 32 * qt + n;
    if (query >= N) continue;
    const float den = (float)(query + 1) + fscale * rs;
    const float inv = p.normalize ? 1.0f / (den + p.eps) : 1.0f;
    if (p.den != nullptr && h == 0) p.den[hrow + query] = den;
    const size_t obase = (hrow + query) * (size_t)dv;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int col = 32 * mt + 8 * g + 4 * h;
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = (fscale * acc[qt][mt][4 * g + e] + vsum[mt][4 * g + e]) * inv;
        if (VEC) {
          if (col < dv) {
            if (p.out_f32) {
              *reinterpret_cast<f32x4*>(static_cast<float*>(p.out) + obase + col) = (f32x4){y[0], y[1], y[2], y[3]};
            } else {
              *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p.out) + obase + col) =
                  (u32x2){pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
            }
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (col + e < dv) {
              if (p.out_f32)
                static_cast<float*>(p.out)[obase + col + e] = y[e];
              else
                static_cast<uint16_t*>(p.out)[obase + col + e] = f32_to_bf16_bits(y[e]);
            }
          }
        }
      }
    }
  }
}

template <int KS, int MT, int QT, bool VEC, bool UNIT, bool DMA>
__global__ __launch_bounds__(256) void based_parallel_bf16_kernel(const ParallelParams p) {
  constexpr int DK = 16 * KS, DV = 32 * MT, BM = 128 * QT, NSNAP = BM / BN;
  constexpr int KROW = DK + 8;
  constexpr int LPR = 256 / DV;
  constexpr int NRAW = 4;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[DMA ? 1 : 2][DMA ? 8 : BN * KROW];
  __shared__ __attribute__((aligned(16))) uint16_t VTs[2][DV * VROW];
  __shared__ __attribute__((aligned(16))) float snap[NSNAP][DV * LPR];
  __shared__ __attribute__((aligned(16))) uint16_t Kraw[DMA ? NRAW : 1][DMA ? BN * 16 : 8];
  __shared__ __attribute__((aligned(16))) uint16_t Vraw[DMA ? NRAW : 1][DMA ? BN * DV : 8];
  based_parallel_body<KS, MT, QT, VEC, UNIT, DMA>(p, Ks, VTs, snap, Kraw, Vraw);
}

template <int KS, int MT, int QT>
int launch_bf16(const ParallelParams& pp, bool vec, hipStream_t stream) {
  constexpr int BM = 128 * QT;
  ParallelParams p = pp;
  p.nqb = (p.N + BM - 1) / BM;
  const dim3 grid((unsigned)(p.nqb * p.BH)), block(256);
  const bool unit = p.inv_c == 1.0f && p.inv_c2 == 1.0f;
  // buffer offsets are 32-bit: one head's K and V must stay below 2^31 bytes
  const bool dma = vec && p.d == 16 && (p.dv % 8) == 0 && (long long)p.N * p.dv * 2 < (1ll << 30);
  if constexpr (KS == 1 && MT <= 2) {
    if (dma && unit) {
      hipLaunchKernelGGL((based_parallel_bf16_kernel<KS, MT, QT, true, true, true>), grid, block, 0, stream, p);
      return (int)hipGetLastError();
    }
    if (dma) {
      hipLaunchKernelGGL((based_parallel_bf16_kernel<KS, MT, QT, true, false, true>), grid, block, 0, stream, p);
      return (int)hipGetLastError();
    }
  }
  if (vec && unit)
    hipLaunchKernelGGL((based_parallel_bf16_kernel<KS, MT, QT, true, true, false>), grid, block, 0, stream, p);
  else if (vec)
    hipLaunchKernelGGL((based_parallel_bf16_kernel<KS, MT, QT, true, false, false>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((based_parallel_bf16_kernel<KS, MT, QT, false, false, false>), grid, block, 0, stream, p);
  return (int)hipGetLastError();
}

template <int KS>
int dispatch_mt(const ParallelParams& p, bool vec, hipStream_t stream) {
  const int dv = p.dv;
  if (dv <= 32) return launch_bf16<KS, 1, 2>(p, vec, stream);
  if (dv <= 64) return launch_bf16<KS, 2, 2>(p, vec, stream);
  return launch_bf16<KS, 4, 1>(p, vec, stream);
}

}  // namespace

int launch_based_parallel_fp32(const ParallelArgs& a, hipStream_t stream);

int launch_based_parallel(const ParallelArgs& a, hipStream_t stream) {
  if (a.in_f32) return launch_based_parallel_fp32(a, stream);
  ParallelParams p{};
  p.q = static_cast<const uint16_t*>(a.q);
  p.k = static_cast<const uint16_t*>(a.k);
  p.v = static_cast<const uint16_t*>(a.v);
  p.out = a.out;
  p.den = a.den;
  p.BH = a.BH;
  p.N = a.N;
  p.d = a.d;
  p.dv = a.dv;
  // Work in u'' = 2^-2k u with u = (q.k + 1/c)^2 - 1/c^2 = (2/c^2) r, k chosen so the weight of
  // "1", W = 2^-2k * 2/c^2, is close to 1 (u'' ~ r).
  const double ic = 1.0 / (double)a.scale;
  const int k = (int)__builtin_lround(0.5 * __builtin_log2(2.0 * ic * ic) - 0.25);
  const double qs = __builtin_ldexp(1.0, -k);
  const float icf = (float)(ic * qs);
  p.qscale = (float)qs;
  p.inv_c = icf;
  p.inv_c2 = (float)((double)icf * (double)icf);
  const double w = 2.0 * (double)icf * (double)icf;   // weight of "1" in u'' units
  p.fscale = (float)(1.0 / w);
  const _Float16 whi = (_Float16)w;
  const _Float16 wlo = (_Float16)(w - (double)whi);
  const u32 hb = __builtin_bit_cast(uint16_t, whi), lb = __builtin_bit_cast(uint16_t, wlo);
  p.ones_hi = hb | (hb << 16);
  p.ones_lo = ((double)wlo == 0.0) ? 0u : (lb | (lb << 16));
  p.eps = a.eps;
  p.normalize = a.normalize ? 1 : 0;
  p.out_f32 = a.out_f32 ? 1 : 0;
  const bool vec = (a.d % 8 == 0) && (a.dv % 4 == 0) && ((reinterpret_cast<uintptr_t>(a.q) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(a.k) & 15) == 0) && ((reinterpret_cast<uintptr_t>(a.v) & 7) == 0) &&
                   ((reinterpret_cast<uintptr_t>(a.out) & 15) == 0);
  if (a.d <= 16) return dispatch_mt<1>(p, vec, stream);
  if (a.d <= 32) return dispatch_mt<2>(p, vec, stream);
  if (a.d <= 64) return dispatch_mt<4>(p, vec, stream);
  return dispatch_mt<8>(p, vec, stream);
}

}  // namespace la
