// Shared device helpers for the MI355X (gfx950) MegaGate/MegaMoE kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define MI355_DEV __device__ __forceinline__
#define MI355_HD __host__ __device__ __forceinline__

typedef __attribute__((ext_vector_type(2))) int v2i;
typedef __attribute__((ext_vector_type(4))) int v4i;
typedef __attribute__((ext_vector_type(8))) int v8i;
typedef __attribute__((ext_vector_type(4))) short v4s;
typedef __attribute__((ext_vector_type(4))) float v4f;
typedef __attribute__((ext_vector_type(16))) float v16f;
typedef __attribute__((ext_vector_type(8))) __bf16 v8bf;

#define LDS_PTR(T, p) ((__attribute__((address_space(3))) T*)(p))

// ---- bit casts usable in host code too (the host-side checker under tests/native runs the GEMM
// epilogues on the CPU); the device compile keeps the HIP intrinsics
MI355_HD uint32_t f32_bits(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __float_as_uint(f);
#else
  return __builtin_bit_cast(uint32_t, f);
#endif
}
MI355_HD float bits_f32(uint32_t u) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __uint_as_float(u);
#else
  return __builtin_bit_cast(float, u);
#endif
}

// ---- bf16 <-> f32 (round to nearest even, NaN kept quiet) -------------------------------
MI355_HD float bf16_to_f32(uint16_t b) { return bits_f32(((uint32_t)b) << 16); }
MI355_HD uint16_t f32_to_bf16(float f) {
  const uint32_t u = f32_bits(f);
  const uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  return (uint16_t)(((u & 0x7fffffffu) > 0x7f800000u) ? ((u >> 16) | 0x40u) : r);  // select, no branch
}

// ---- OCP MX e4m3fn / e8m0 --------------------------------------------------------------
// float -> e4m3fn, round to nearest even, saturating to +-448 (0x7e / 0xfe).
MI355_HD uint32_t f32_to_e4m3(float v) {
  uint32_t sign = (f32_bits(v) >> 24) & 0x80u;
  float a = fminf(fabsf(v), 448.0f);
  uint32_t code;
  if (a < 0.015625f) {                 // below 2^-6: subnormal grid of 2^-9
    code = (uint32_t)rintf(a * 512.0f);  // 0..8 (8 == smallest normal, code 0x08)
  } else {
    uint32_t bits = f32_bits(a);
    int32_t e = (int32_t)(bits >> 23) - 127;
    uint32_t mant = bits & 0x7fffffu;
    uint32_t m3 = mant >> 20, rem = mant & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (m3 & 1u))) m3++;
    if (m3 == 8u) { m3 = 0; e++; }
    code = ((uint32_t)(e + 7) << 3) | m3;
  }
  return sign | code;
}
// Shared exponent of a 32-element block as e8m0 code: the smallest e with amax <= 448 * 2^e (the
// reference's MX scale algorithm 1, so no element saturates). With amax = M * 2^E, M in [1, 2),
// 448 * 2^(E-8) = 1.75 * 2^E: e = E - 8 for M <= 1.75 (mantissa bits <= 0x600000), E - 7 above.
// Clamped to [-127, 127]; all-zero (and fp32-subnormal) blocks get 2^-127.
MI355_HD uint32_t mx_scale_code(float amax) {
  if (!(amax > 0.0f)) return 0u;
  const uint32_t bits = f32_bits(amax);
  const int32_t E = (int32_t)((bits >> 23) & 0xff) - 127;
  if (E == -127) return 0u;
  int32_t s = E - 8 + ((bits & 0x7fffffu) > 0x600000u ? 1 : 0);
  if (s < -127) s = -127;
  if (s > 127) s = 127;
  return (uint32_t)(s + 127);
}
// e4m3fn code of v with |v| <= 448 (an element scaled by mx_scale_code's exponent): the hardware
// conversion (round to nearest even), equal to f32_to_e4m3 on that range.
MI355_DEV uint32_t f32_to_e4m3_inrange(float v) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v, 0.0f, 0, false) & 0xffu;
}
// Multiply by 2^-(code-127) exactly (power-of-two scaling).
MI355_HD float mx_apply_inv_scale(float v, uint32_t code) { return ldexpf(v, 127 - (int)code); }

// ---- wave helpers -----------------------------------------------------------------------
MI355_DEV float wave_shfl_xor(float v, int m) { return __shfl_xor(v, m, 64); }
MI355_DEV int wave_shfl_xor(int v, int m) { return __shfl_xor(v, m, 64); }

// Error codes shared with the C ABI.
#define MI355MOE_OK 0
#define MI355MOE_EINVAL -1
#define MI355MOE_ELAUNCH -2
#define MI355MOE_EUNSUPPORTED -3
#define MI355MOE_EWORKSPACE -4
