// Device helpers shared by the prologue and the main loop (gfx950 / CDNA4, wave64).
//
// Numerics rules that every quantizer in this library follows, because the quantized tensors must
// be bit-exact with the reference scheme:
//   * fp32 division is correctly rounded (`__fdiv_rn`); the library is never built with fast-math;
//   * rounding to an integer is round-half-to-even (`rintf` -> v_rndne_f32), then clamped;
//   * fp32 -> e4m3 goes through v_cvt_pk_fp8_f32 (OCP e4m3fn, round-to-nearest-even on gfx950);
//   * no fused multiply-add is formed where the scheme has two roundings: every such expression has
//     no addition (a*b*c), so contraction cannot apply.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sage {

typedef uint8_t u8;
typedef uint32_t u32;
typedef uint64_t u64;
typedef _Float16 f16;
typedef __bf16 bf16;

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int HD = 128;          // the largest head_dim served (64 is the other)
constexpr int NPAD = 64;         // N_pad granule
constexpr float P_SCALE = 448.0f;
constexpr float I8_MAX = 127.0f;
constexpr float SCALE_FLOOR = 1e-12f;
constexpr float LOG2E_F = 1.4426950408889634f;

// 16-bit element widen. bf16 -> fp32 and fp16 -> fp32 are exact.
__device__ __forceinline__ float widen(f16 x) { return (float)x; }
__device__ __forceinline__ float widen(bf16 x) { return (float)x; }

// Unpack 8 16-bit elements held in a 16-byte vector.
template <typename T>
__device__ __forceinline__ void unpack8(const u32x4 w, float* out) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t x = w[i];
    const uint16_t lo = (uint16_t)(x & 0xffffu), hi = (uint16_t)(x >> 16);
    T a, b;
    __builtin_memcpy(&a, &lo, 2);
    __builtin_memcpy(&b, &hi, 2);
    out[2 * i] = widen(a);
    out[2 * i + 1] = widen(b);
  }
}

// Two fp32 -> two e4m3 bytes in the low 16 bits (byte 0 = a).
__device__ __forceinline__ uint32_t fp8x2(float a, float b) {
  return ((uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false)) & 0xffffu;
}
// Four fp32 -> four e4m3 bytes, memory order a, b, c, d.
__device__ __forceinline__ uint32_t fp8x4(float a, float b, float c, float d) {
  // The first convert writes the low half-word and keeps the high half of its "old" operand,
  // which the second convert overwrites, so any value does: passing a's own bits lets the
  // convert write over a's register instead of a zeroed copy.
  int r = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, __float_as_int(a), false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, r, true);
}

// Round half to even, clamp to [-128, 127], return the int8 byte.
__device__ __forceinline__ uint32_t i8_rne(float x) {
  const float r = fminf(fmaxf(__builtin_rintf(x), -128.0f), 127.0f);
  return ((uint32_t)(int)r) & 0xffu;
}
// Four already-quantizable fp32 -> four int8 bytes (memory order a, b, c, d).
__device__ __forceinline__ uint32_t i8x4(float a, float b, float c, float d) {
  return i8_rne(a) | (i8_rne(b) << 8) | (i8_rne(c) << 16) | (i8_rne(d) << 24);
}

// RN(x / s) from y = RN(1 / s), in three operations instead of a full division: q = RN(x*y) is
// within an ulp of x/s, e = RN(q*s - x) is then exact (one fma), and RN(q - e*y) is the correctly
// rounded quotient (Markstein's theorem for round-to-nearest with a correctly rounded reciprocal).
// The bits equal __fdiv_rn(x, s) for normal quotients; signed zeros pass through (-0 / s = -0).
// The quantizers call it with one reciprocal per row (or a constant divisor), so a row of D
// quotients costs one full division.
__device__ __forceinline__ float div_by(float x, float s, float y) {
  const float q = x * y;
  const float e = __builtin_fmaf(q, s, -x);
  return __builtin_fmaf(-e, y, q);
}
constexpr float RCP_P_SCALE = 1.0f / 448.0f;   // RN(1/448)
constexpr float RCP_I8_MAX = 1.0f / 127.0f;    // RN(1/127)

// One DPP lane move within each 16-lane row (ctrl: quad_perm / row_mirror / row_half_mirror).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Max over the G lanes of an aligned G-lane group (G = 8 or 16: lanes Gg .. Gg+G-1), as DPP
// moves folded into v_max_f32: xor 1 and xor 2 (quad_perm), then the mirrored lane of the
// 8-lane half-row (the other quad) and of the 16-lane row (the other half).
template <int G = 16>
__device__ __forceinline__ float maxg(float x) {
  x = fmaxf(x, dpp_mov<0xB1>(x));    // quad_perm [1,0,3,2]
  x = fmaxf(x, dpp_mov<0x4E>(x));    // quad_perm [2,3,0,1]
  x = fmaxf(x, dpp_mov<0x141>(x));   // row_half_mirror
  if (G == 16) x = fmaxf(x, dpp_mov<0x140>(x));   // row_mirror
  return x;
}

}  // namespace sage
