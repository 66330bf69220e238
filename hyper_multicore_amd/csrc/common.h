// Shared device helpers for the MI355X (gfx950) MegaGate/MegaMoE kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define MI355_DEV __device__ __forceinline__

typedef __attribute__((ext_vector_type(2))) int v2i;
typedef __attribute__((ext_vector_type(4))) int v4i;
typedef __attribute__((ext_vector_type(8))) int v8i;
typedef __attribute__((ext_vector_type(4))) short v4s;
typedef __attribute__((ext_vector_type(4))) float v4f;
typedef __attribute__((ext_vector_type(16))) float v16f;
typedef __attribute__((ext_vector_type(8))) __bf16 v8bf;

#define LDS_PTR(T, p) ((__attribute__((address_space(3))) T*)(p))

// ---- bf16 <-> f32 (round to nearest even, NaN kept quiet) -------------------------------
MI355_DEV float bf16_to_f32(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }
MI355_DEV uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// ---- OCP MX e4m3fn / e8m0 --------------------------------------------------------------
// float -> e4m3fn, round to nearest even, saturating to +-448 (0x7e / 0xfe).
MI355_DEV uint32_t f32_to_e4m3(float v) {
  uint32_t sign = (__float_as_uint(v) >> 24) & 0x80u;
  float a = fminf(fabsf(v), 448.0f);
  uint32_t code;
  if (a < 0.015625f) {                 // below 2^-6: subnormal grid of 2^-9
    code = (uint32_t)rintf(a * 512.0f);  // 0..8 (8 == smallest normal, code 0x08)
  } else {
    uint32_t bits = __float_as_uint(a);
    int32_t e = (int32_t)(bits >> 23) - 127;
    uint32_t mant = bits & 0x7fffffu;
    uint32_t m3 = mant >> 20, rem = mant & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (m3 & 1u))) m3++;
    if (m3 == 8u) { m3 = 0; e++; }
    code = ((uint32_t)(e + 7) << 3) | m3;
  }
  return sign | code;
}
// Shared-exponent of a 32-element block (OCP MX v1.0): floor(log2(amax)) - 8, as e8m0 code.
MI355_DEV uint32_t mx_scale_code(float amax) {
  if (!(amax > 0.0f)) return 0u;  // all-zero block: any scale; use 2^-127
  int32_t e = (int32_t)((__float_as_uint(amax) >> 23) & 0xff) - 127;  // floor(log2) for normals
  if (e == -127) e = -127;                                               // fp32 denormal amax
  int32_t s = e - 8;
  if (s < -127) s = -127;
  if (s > 127) s = 127;
  return (uint32_t)(s + 127);
}
// Multiply by 2^-(code-127) exactly (power-of-two scaling).
MI355_DEV float mx_apply_inv_scale(float v, uint32_t code) { return ldexpf(v, 127 - (int)code); }

// ---- wave helpers -----------------------------------------------------------------------
MI355_DEV float wave_shfl_xor(float v, int m) { return __shfl_xor(v, m, 64); }
MI355_DEV int wave_shfl_xor(int v, int m) { return __shfl_xor(v, m, 64); }

// Error codes shared with the C ABI.
#define MI355MOE_OK 0
#define MI355MOE_EINVAL -1
#define MI355MOE_ELAUNCH -2
#define MI355MOE_EUNSUPPORTED -3
