// Shared device helpers for the gfx950 BASED kernels: vector types, bf16 packing, MFMA
// wrappers and the 32x32 accumulator layout.
//
// MFMA layout used throughout (v_mfma_f32_32x32x16_bf16, wave64):
//   A (32 x 16): lane l holds row l%32, k = 8*(l/32) .. +7
//   B (16 x 32): lane l holds col l%32, k = 8*(l/32) .. +7
//   C (32 x 32): lane l holds col l%32, rows 8*(i/4) + 4*(l/32) + (i%4) for i = 0..15
// Only the pairing "element e of lane group h in A with element e of lane group h in B" is
// relied on for the contraction index, so any K permutation applied to both operands is fine.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace la {

typedef uint32_t u32;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(u32)))) u32 u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(u32)))) u32 u32x2;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;

constexpr int kWave = 64;

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 f16x2;

// float pair -> packed fp16, round to nearest even (v_cvt_pk_f16_f32).
__device__ __forceinline__ u32 pack_f16x2(float lo, float hi) {
  f16x2 p = __builtin_convertvector((f32x2){lo, hi}, f16x2);
  return __builtin_bit_cast(u32, p);
}

// (x0*x0 + c, x1*x1 + c) as packed fp16, each rounded once from the exact product-sum
// (the compiler selects v_fma_mixlo_f16 / v_fma_mixhi_f16 for the scalar conversions).
__device__ __forceinline__ u32 sq_plus_f16x2(float x0, float x1, float c) {
  const f16x2 r = {(_Float16)__builtin_fmaf(x0, x0, c), (_Float16)__builtin_fmaf(x1, x1, c)};
  return __builtin_bit_cast(u32, r);
}

__device__ __forceinline__ float f16_lo_to_f32(u32 w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
}
__device__ __forceinline__ float f16_hi_to_f32(u32 w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16)); }

// sum += a.lo*b.lo + a.hi*b.hi over packed fp16 pairs, fp32 accumulate (v_dot2_f32_f16).
__device__ __forceinline__ float dot2_f16(u32 a, u32 b, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), acc, false);
}

__device__ __forceinline__ f32x16 mfma32x32x16_f16(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                0, 0, 0);
}

// v_mfma_f32_16x16x32_bf16.  A (16 x 32): lane l holds row l%16, k = 8*(l/16) .. +7; B likewise
// with col l%16; C (16 x 16): lane l holds col l%16, rows 4*(l/16) + i for i = 0..3.
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

// Packed fp16 a*b + c, one rounding per half (v_pk_fma_f16).
__device__ __forceinline__ u32 pk_fma_f16(u32 a, u32 b, u32 c) {
  return __builtin_bit_cast(u32, __builtin_elementwise_fma(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b),
                                                           __builtin_bit_cast(f16x2, c)));
}
__device__ __forceinline__ u32 pk_mul_f16(u32 a, u32 b) {
  return __builtin_bit_cast(u32, __builtin_bit_cast(f16x2, a) * __builtin_bit_cast(f16x2, b));
}

// float -> bf16 bits, round to nearest even (the hardware conversion on gfx950).
__device__ __forceinline__ u32 pack_bf16x2(float lo, float hi) {
  bf16x2 p = __builtin_convertvector((f32x2){lo, hi}, bf16x2);
  return __builtin_bit_cast(u32, p);
}

__device__ __forceinline__ float bf16_lo_to_f32(u32 w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16_hi_to_f32(u32 w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __builtin_bit_cast(float, (u32)b << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return (uint16_t)(pack_bf16x2(f, 0.f) & 0xffffu);
}

// sum += a.lo*b.lo + a.hi*b.hi over packed bf16 pairs, fp32 accumulate (v_dot2c_f32_bf16).
__device__ __forceinline__ float dot2_bf16(u32 a, u32 b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), acc,
                                         false);
}

__device__ __forceinline__ f32x16 mfma32x32x16(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

// Multiplies 8 packed bf16 values by a power of two (exact unless the result leaves the
// bf16 range).
__device__ __forceinline__ u32x4 scale_bf16x8(u32x4 x, float s) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = pack_bf16x2(bf16_lo_to_f32(x[i]) * s, bf16_hi_to_f32(x[i]) * s);
  return r;
}

__device__ __forceinline__ f32x16 splat16(float x) {
  f32x16 r;
#pragma unroll
  for (int i = 0; i < 16; ++i) r[i] = x;
  return r;
}

// Wave-wide maximum of an unsigned value (fp32 magnitudes order as their bits), returned in
// every lane: a running maximum along each row of 16 lanes (DPP row_shr 1, 2, 4, 8), then rows
// 0-1 and 2-3 joined by row_bcast15 and all four by row_bcast31, read from lane 63.  Lanes
// whose DPP source lies outside the row take 0, which leaves a maximum of unsigned values alone.
__device__ __forceinline__ u32 wave_max_u32(u32 x) {
  x = max(x, (u32)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xf, 0xf, false));   // row_shr:1
  x = max(x, (u32)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xf, 0xf, false));   // row_shr:2
  x = max(x, (u32)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xf, 0xf, false));   // row_shr:4
  x = max(x, (u32)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xf, 0xf, false));   // row_shr:8
  x = max(x, (u32)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xa, 0xf, false));   // row_bcast:15
  x = max(x, (u32)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xc, 0xf, false));   // row_bcast:31
  return (u32)__builtin_amdgcn_readlane((int)x, 63);
}

// Row (key / dv index) of element i of a 32x32 accumulator held by lane group h.
__device__ __forceinline__ int c32_row(int i, int h) { return 8 * (i >> 2) + 4 * h + (i & 3); }

// ---- global -> LDS copies (buffer_load_dwordx4 ... lds)
//
// A raw buffer descriptor over [base, base + bytes): stride 0, num_records in bytes; dword 3
// selects raw (untyped) addressing with per-dword range checking, so bytes at or past the end
// read as zero.  base and bytes must be wave-uniform.
__device__ __forceinline__ u32x4 buffer_rsrc(const void* base, u32 bytes) {
  const unsigned long long a = reinterpret_cast<unsigned long long>(base);
  return (u32x4){(u32)__builtin_amdgcn_readfirstlane((int)(u32)a),
                 (u32)__builtin_amdgcn_readfirstlane((int)(u32)(a >> 32)) & 0xffffu,
                 (u32)__builtin_amdgcn_readfirstlane((int)bytes), 0x00020000u};
}

// Lane i copies the 16 bytes at byte offset voff of the buffer to LDS address lds_base + 16 i
// (lds_base wave-uniform).  Issued as inline assembly so that the compiler's wait-count pass does
// not treat every later LDS read as dependent on the copy: the caller orders copies and reads
// itself, with s_waitcnt vmcnt and a barrier.  Each call adds one to the wave's vmcnt.
//
// The compiler inserts no wait states in front of inline assembly, so the copy carries its
// own: a VALU write of an SGPR (v_readfirstlane of the descriptor in buffer_rsrc) needs five
// wait states before a VMEM instruction reads that SGPR, and an SALU write of M0 one before an
// LDS-DMA copy.  s_nop 4 provides five, whatever the scheduler placed just before the copy.
__device__ __forceinline__ void lds_copy16(const u32x4& rsrc, u32 lds_base, int voff) {
  asm volatile(
      "s_nop 4\n\t"
      "buffer_load_dwordx4 %0, %1, 0 offen lds"
      :
      : "v"(voff), "s"(rsrc), "{m0}"(lds_base)
      : "memory");
}

// LDS byte address of a __shared__ object.
template <class T>
__device__ __forceinline__ u32 lds_addr(const T* p) {
  return (u32)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// ---- raw buffer loads / stores
//
// A raw buffer resource over [base, base + bytes) (dword 3 as for buffer_rsrc above): accesses at
// offsets >= bytes read as zero and are dropped on store, which takes the place of per-lane
// bounds checks.  base and bytes must be wave-uniform.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, u32 bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// An offset that is out of range for every resource built by make_rsrc (bytes < 2^31).
constexpr int kOffOutOfRange = 0x7ffffff0;

__device__ __forceinline__ u32x2 buf_load_b64(__amdgpu_buffer_rsrc_t r, int voff) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, 0, 0));
}
__device__ __forceinline__ u32x4 buf_load_b128(__amdgpu_buffer_rsrc_t r, int voff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
}
__device__ __forceinline__ void buf_store_b64(u32x2 x, __amdgpu_buffer_rsrc_t r, int voff) {
  typedef __attribute__((__vector_size__(2 * sizeof(u32)))) u32 v2;
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2, x), r, voff, 0, 0);
}
__device__ __forceinline__ void buf_store_b128(u32x4 x, __amdgpu_buffer_rsrc_t r, int voff) {
  typedef __attribute__((__vector_size__(4 * sizeof(u32)))) u32 v4;
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4, x), r, voff, 0, 0);
}

}  // namespace la
