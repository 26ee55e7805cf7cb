// Shared helpers for the gfx950 kernels and their C-ABI wrappers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/selas_amd.h"

namespace selas {

// ------------------------------------------------------------------ host side

// Records a formatted message for selas_last_error() and returns `code`.
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the message and returns SELAS_OK.
int ok();
// Turns the launch status of the last kernel into a return code.
int check_launch(const char *what);

inline bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline bool valid_dtype(int dt) { return dt == SELAS_F32 || dt == SELAS_F16 || dt == SELAS_BF16; }
inline const char *dtype_name(int dt) {
  return dt == SELAS_F32 ? "f32" : dt == SELAS_F16 ? "f16" : dt == SELAS_BF16 ? "bf16" : "?";
}

// The 16-entry codebook, passed by value so that it lives in scalar registers.
struct Code16 {
  float v[16];
};

// ------------------------------------------------------------------ device side

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
  return __builtin_amdgcn_perm(s0, s1, sel);
}

// Raw buffer resource over `bytes` bytes (gfx9 descriptor word 3: 0x00020000).
// Loads past the range return zeros and stores past it are dropped.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), static_cast<short>(0), static_cast<int>(bytes),
                                           0x00020000);
}
__device__ __forceinline__ uint4 load_b128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ float load_f32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
// 16 bytes per lane from a buffer straight into LDS: lane i writes lds + 16*i.
__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t r, uint8_t *lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16, voff, soff, 0, 0);
}

// D(32x32) += A(32x16) B(16x32) in bf16 with fp32 accumulation. Lane l supplies
// A[l % 32][8*(l/32) .. +8] and B[8*(l/32) .. +8][l % 32]; it holds
// D[8*(r/4) + 4*(l/32) + r%4][l % 32] in register r.
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// s_waitcnt with only the vector-memory counter limited to N (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// GELU with the tanh approximation, x * 0.5 * (1 + tanh(z)), z = sqrt(2/pi) *
// (x + 0.044715 x^3), through 0.5 * (1 + tanh(z)) = 1 / (1 + exp(-2z)) =
// 1 / (1 + 2^u), u = x (A + B x^2), A = -2 log2(e) sqrt(2/pi), B = 0.044715 A:
// one multiply, one fused multiply-add, one multiply, then one hardware
// base-2 exponential and one reciprocal instead of tanhf (a few ulp of fp32,
// below the rounding to a 16-bit output). One definition serves the segment
// kernels and the GEMM epilogue, so both give the same bits.
__device__ __forceinline__ float gelu_tanh_fast(float x) {
  constexpr float kA = -2.302208198144325f;   // -2 log2(e) sqrt(2 / pi)
  constexpr float kB = -0.1029432395800235f;  // 0.044715 kA
  const float u = x * __builtin_fmaf(kB, x * x, kA);
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(u));
}

// fp32 -> bf16 bits, round to nearest even (the rounding torch uses for
// bfloat16 casts). Any NaN becomes the quiet NaN 0x7FC0.
__device__ __forceinline__ uint16_t bf16_bits_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7FC0;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// Returns `v` unchanged but opaque to the optimiser (no instruction is
// emitted): a conversion of the result can then not be merged with the
// arithmetic that produced `v` (for example fp16(a * b) into one
// mixed-precision FMA that rounds the exact product once).
__device__ __forceinline__ float materialize(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

// fp32 -> fp16 bits, IEEE round to nearest even (overflow to inf, gradual
// underflow), done by the hardware convert on the already-rounded fp32 value.
__device__ __forceinline__ uint16_t f16_bits_rne(float f) {
  _Float16 h = static_cast<_Float16>(materialize(f));
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }
__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  return static_cast<float>(__builtin_bit_cast(_Float16, b));
}

// Loads element i of a 16-bit or 32-bit float array as fp32.
template <int DT>
__device__ __forceinline__ float load_f(const void *p, int64_t i) {
  if constexpr (DT == SELAS_F32) return static_cast<const float *>(p)[i];
  else if constexpr (DT == SELAS_F16) return f16_bits_to_f32(static_cast<const uint16_t *>(p)[i]);
  else return bf16_bits_to_f32(static_cast<const uint16_t *>(p)[i]);
}

// Rounds fp32 to the storage type DT and stores element i.
template <int DT>
__device__ __forceinline__ void store_f(void *p, int64_t i, float v) {
  if constexpr (DT == SELAS_F32) static_cast<float *>(p)[i] = v;
  else if constexpr (DT == SELAS_F16) static_cast<uint16_t *>(p)[i] = f16_bits_rne(v);
  else static_cast<uint16_t *>(p)[i] = bf16_bits_rne(v);
}

// Two fp32 values -> packed (lo, hi) bf16 pair with the gfx950 hardware convert
// (round to nearest even; identical to bf16_bits_rne for every non-NaN value).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 v = {static_cast<__bf16>(materialize(lo)), static_cast<__bf16>(materialize(hi))};
  return __builtin_bit_cast(uint32_t, v);
}

// GELU of two values rounded as a packed bf16 pair (the hardware convert).
__device__ __forceinline__ uint32_t gelu_bf16x2(float lo, float hi) {
  return pack_bf16x2(gelu_tanh_fast(lo), gelu_tanh_fast(hi));
}

// Wave-wide (64 lanes) reductions through the cross-lane network.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace selas
