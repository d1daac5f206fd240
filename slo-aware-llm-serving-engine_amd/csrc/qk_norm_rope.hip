// Fused per-head RMSNorm of q and k, rotary embedding, and the slot-mapped
// KV-cache write (gfx950).
//
// Replaces, in one pass over the fused QKV projection output, the steps of
// Qwen3Attention.forward between the projection and the attention call
// (nanovllm/models/qwen3.py:80-86): q_norm / k_norm (nanovllm/layers/
// layernorm.py:16-26), rotary_emb (nanovllm/layers/rotary_embedding.py:6-14,
// 37-48) and the store_kvcache that Attention.forward issues first
// (nanovllm/layers/attention.py:10-40, 59-66), so q and k make one round trip
// through HBM instead of four.  Arithmetic follows the reference's rounding
// points:
//   RMSNorm  var = mean(x^2) in fp32 (here: the exact mean, rounded once),
//            r = rsqrt(var + eps) in fp32 (here: correctly rounded),
//            n = bf16(x * r), out = bf16(n * w)
//   RoPE     x1, x2 = halves of out (as fp32); y1 = x1*cos - x2*sin,
//            y2 = x2*cos + x1*sin, each product and sum rounded in fp32 (no
//            fused multiply-add), then bf16
// K is stored after RoPE (docs/project_manual.md:539); V is stored as given.
// E4M3FN pools use the quantisation of the store kernel.
//
// One 16-lane group per (token, head) of the QKV row; lane j holds elements
// 8j..8j+7 (one 16-byte load), so a head's statistics are a 16-lane
// reduction and the RoPE partner of element d (d +- 64) sits in lane j ^ 8.
#include "common.h"
#include "capi_internal.h"

namespace slo {

constexpr int QK_HD = 128;

__device__ __forceinline__ float bf16_round(float f) { return __uint_as_float(f32_to_bf16_bits(f) << 16); }

__global__ void __launch_bounds__(256)
qk_norm_rope_store_kernel(const uint16_t* __restrict__ qkv, int64_t qkv_stride, const int64_t* __restrict__ positions,
                          int64_t units, int num_heads, int num_kv_heads, const uint16_t* __restrict__ q_w,
                          const uint16_t* __restrict__ k_w, float eps, const float* __restrict__ cos_sin,
                          int max_position, uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_out,
                          const int32_t* __restrict__ slot_mapping, int kv_dtype, void* __restrict__ k_cache,
                          void* __restrict__ v_cache, float* __restrict__ k_scale, float* __restrict__ v_scale,
                          int64_t num_slots, float scale_floor) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int j = lane & 15;
  const int64_t u = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  if (u >= units) return;  // whole 16-lane groups leave together
  const int heads = num_heads + 2 * num_kv_heads;
  const int64_t tok = u / heads;
  const int hh = (int)(u % heads);
  const bool is_q = hh < num_heads, is_k = !is_q && hh < num_heads + num_kv_heads;
  const int d0 = 8 * j;

  const u32x4 x = *reinterpret_cast<const u32x4*>(qkv + tok * qkv_stride + (int64_t)hh * QK_HD + d0);
  float f[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_bits_to_f32(x[i] & 0xffffu);
    f[2 * i + 1] = bf16_bits_to_f32(x[i] >> 16);
  }

  const int64_t slot = slot_mapping[tok];
  const bool store = slot >= 0 && slot < num_slots;
  const int kvh = is_k ? hh - num_heads : hh - num_heads - num_kv_heads;

  if (is_q || is_k) {
    // Sum of squares in fp64: every square of a bf16 value is exact and so,
    // for vectors spanning less than 2^15 in magnitude, is the sum, so the
    // mean is rounded to fp32 once whatever the summation order.
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += (double)f[i] * (double)f[i];
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) ss += __shfl_xor(ss, m, 64);
    const float var = (float)(ss / QK_HD);
    const float r = (float)(1.0 / sqrt((double)(var + eps)));
    const uint16_t* w = is_q ? q_w : k_w;
    const u32x4 wv = *reinterpret_cast<const u32x4*>(w + d0);
    float n[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      n[2 * i] = bf16_round(bf16_round(f[2 * i] * r) * bf16_bits_to_f32(wv[i] & 0xffffu));
      n[2 * i + 1] = bf16_round(bf16_round(f[2 * i + 1] * r) * bf16_bits_to_f32(wv[i] >> 16));
    }
    int64_t pos = positions[tok];
    pos = pos < 0 ? 0 : (pos >= max_position ? max_position - 1 : pos);
    const float* cs = cos_sin + pos * QK_HD + (d0 & 63);
    const f32x4 c0 = *reinterpret_cast<const f32x4*>(cs), c1 = *reinterpret_cast<const f32x4*>(cs + 4);
    const f32x4 s0 = *reinterpret_cast<const f32x4*>(cs + 64), s1 = *reinterpret_cast<const f32x4*>(cs + 68);
    const float c[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
    const float s[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float other = __shfl_xor(n[i], 8, 64);  // element d +- 64
      const float a = n[i] * c[i], b = other * s[i];
      y[i] = bf16_round(j < 8 ? a - b : a + b);     // lanes 0-7: x1 half, lanes 8-15: x2 half
    }
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (__float_as_uint(y[2 * i]) >> 16) | (__float_as_uint(y[2 * i + 1]) & 0xffff0000u);
    if (is_q) {
      *reinterpret_cast<u32x4*>(q_out + (tok * num_heads + hh) * QK_HD + d0) = o;
      return;
    }
    *reinterpret_cast<u32x4*>(k_out + (tok * num_kv_heads + kvh) * QK_HD + d0) = o;
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = y[i];
    if (!store) return;
  } else if (!store) {
    return;
  }
  // K (normalised and rotated) or V (as given) into the pool.
  const int64_t dst = (slot * num_kv_heads + kvh) * QK_HD + d0;
  if (kv_dtype == KV_BF16) {
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (__float_as_uint(f[2 * i]) >> 16) | (__float_as_uint(f[2 * i + 1]) & 0xffff0000u);
    *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(is_k ? k_cache : v_cache) + dst) = o;
  } else {
    float scale;
    const u32x2 codes = e4m3_encode8<16>(f, scale_floor, scale);
    *reinterpret_cast<u32x2*>(static_cast<uint8_t*>(is_k ? k_cache : v_cache) + dst) = codes;
    if (j == 0) (is_k ? k_scale : v_scale)[slot * num_kv_heads + kvh] = scale;
  }
}

}  // namespace slo

using namespace slo;

extern "C" int slo_qk_norm_rope_store(const void* qkv, int64_t qkv_row_stride, const int64_t* positions,
                                      int32_t num_tokens, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                      const void* q_norm_weight, const void* k_norm_weight, float eps,
                                      const float* cos_sin, int32_t max_position, void* q_out, void* k_out,
                                      const int32_t* slot_mapping, int32_t kv_dtype, void* k_cache, void* v_cache,
                                      float* k_scale, float* v_scale, int64_t num_slots, float scale_floor,
                                      slo_stream_t stream) {
  if (num_tokens < 0 || num_heads <= 0 || num_kv_heads <= 0)
    return fail(SLO_ERR_INVALID, "qk_norm_rope_store: bad token/head count");
  if (head_dim != QK_HD) return fail(SLO_ERR_UNSUPPORTED, "qk_norm_rope_store: head_dim must be 128");
  if (kv_dtype != KV_BF16 && kv_dtype != KV_FP8_E4M3FN) return fail(SLO_ERR_INVALID, "qk_norm_rope_store: bad kv_dtype");
  if (max_position <= 0) return fail(SLO_ERR_INVALID, "qk_norm_rope_store: max_position must be positive");
  if (num_tokens == 0) return SLO_OK;
  if (!qkv || !positions || !q_norm_weight || !k_norm_weight || !cos_sin || !q_out || !k_out || !slot_mapping ||
      !k_cache || !v_cache)
    return fail(SLO_ERR_INVALID, "qk_norm_rope_store: null pointer");
  if (kv_dtype == KV_FP8_E4M3FN && (!k_scale || !v_scale))
    return fail(SLO_ERR_INVALID, "qk_norm_rope_store: FP8 needs scale pools");
  if (kv_dtype == KV_FP8_E4M3FN && !(scale_floor > 0.0f))
    return fail(SLO_ERR_INVALID, "qk_norm_rope_store: scale_floor must be > 0");
  if (!(eps >= 0.0f)) return fail(SLO_ERR_INVALID, "qk_norm_rope_store: eps must be >= 0");
  if ((qkv_row_stride % 8) || qkv_row_stride < (int64_t)(num_heads + 2 * num_kv_heads) * head_dim ||
      (reinterpret_cast<uintptr_t>(qkv) % 16) || (reinterpret_cast<uintptr_t>(q_out) % 16) ||
      (reinterpret_cast<uintptr_t>(k_out) % 16) || (reinterpret_cast<uintptr_t>(k_cache) % 16) ||
      (reinterpret_cast<uintptr_t>(v_cache) % 16) || (reinterpret_cast<uintptr_t>(cos_sin) % 16) ||
      (reinterpret_cast<uintptr_t>(q_norm_weight) % 16) || (reinterpret_cast<uintptr_t>(k_norm_weight) % 16))
    return fail(SLO_ERR_INVALID, "qk_norm_rope_store: rows and tables must be 16-byte aligned");
  const int64_t units = (int64_t)num_tokens * (num_heads + 2 * num_kv_heads);
  const int64_t blocks = (units + 15) / 16;
  if (blocks > 0x7fffffff) return fail(SLO_ERR_UNSUPPORTED, "qk_norm_rope_store: too many tokens");
  hipLaunchKernelGGL(qk_norm_rope_store_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(qkv), qkv_row_stride, positions, units, num_heads, num_kv_heads,
                     static_cast<const uint16_t*>(q_norm_weight), static_cast<const uint16_t*>(k_norm_weight), eps,
                     cos_sin, max_position, static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_out), slot_mapping,
                     kv_dtype, k_cache, v_cache, k_scale, v_scale, num_slots, scale_floor);
  return check_launch("qk_norm_rope_store");
}
