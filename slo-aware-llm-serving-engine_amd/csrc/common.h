// Shared device helpers for the gfx950 (CDNA4) attention path.
//
// Layout facts these helpers rely on were checked on gfx950 silicon:
//  * v_mfma_f32_16x16x32_bf16: lane l holds A[m=l%16][k=(l/16)*8+j] and
//    B[k=(l/16)*8+j][n=l%16] (j=0..7); the 4 accumulators of lane l are
//    C[m=(l/16)*4+i][n=l%16].
//  * ds_read_b64_tr_b16: inside each 16-lane group, source lane s supplies an
//    8-byte address; destination lane i receives element (i%4) of the 8-byte
//    rows fetched by source lanes i/4, i/4+4, i/4+8, i/4+12.
//  * v_cvt_pk_f32_fp8 / v_cvt_pk_fp8_f32 use the OCP E4M3FN format; the
//    encode rounds to nearest-even and matches a software RNE encoder on every
//    finite input in [-448, 448].
//  * fp32 '/' in device code is IEEE correctly rounded (hipcc default).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace slo {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) short s16x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

// KV element formats accepted by the C-ABI.
enum KvDtype : int { KV_BF16 = 0, KV_FP8_E4M3FN = 1 };

constexpr float kFp8Max = 448.0f;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits (inputs are finite in this path).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;

// Two fp32 -> packed bf16, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// Decode 4 E4M3FN bytes (one dword) to 4 bf16 (two dwords), byte i to
// element i.  Every E4M3FN value is exactly representable in bf16;
// v_cvt_scalef32_pk_bf16_fp8 converts two bytes per instruction, and with a
// scale of 1.0 (the instruction applies the scale's power of two) it returns
// exactly the bf16 of cvt_pk_f32_fp8's float for all 65,536 byte pairs
// (checked on gfx950 against the two-step float path).
__device__ __forceinline__ u32x2 fp8x4_to_bf16x4(uint32_t w) {
  u32x2 r;
  r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
  r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true));
  return r;
}

__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 as_bf16x8(const u32x4& v) {
  return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ float wave_max_xor(float v, int mask) {
  return fmaxf(v, __shfl_xor(v, mask, 64));
}

// E4M3FN codes of this lane's 8 values of one (token, kv head) vector held by
// GROUP adjacent lanes (the quantisation contract of
// docs/project_manual.md:527-537): amax over the vector (cross-lane), scale =
// amax == 0 ? 1 : max(amax / 448, scale_floor) (correctly rounded division),
// code = E4M3FN_RNE(clamp(x / scale, -448, 448)).  Returns the 8 code bytes
// and the scale.
template <int GROUP>
__device__ __forceinline__ u32x2 e4m3_encode8(const float (&f)[8], float scale_floor, float& scale) {
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(f[j]));
#pragma unroll
  for (int mask = 1; mask < GROUP; mask <<= 1) amax = wave_max_xor(amax, mask);
  scale = amax == 0.0f ? 1.0f : fmaxf(amax / kFp8Max, scale_floor);
  float y[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) y[j] = fminf(fmaxf(f[j] / scale, -kFp8Max), kFp8Max);
  uint32_t w0 = 0, w1 = 0;
  w0 = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], w0, false);
  w0 = __builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], w0, true);
  w1 = __builtin_amdgcn_cvt_pk_fp8_f32(y[4], y[5], w1, false);
  w1 = __builtin_amdgcn_cvt_pk_fp8_f32(y[6], y[7], w1, true);
  return u32x2{w0, w1};
}

}  // namespace slo
