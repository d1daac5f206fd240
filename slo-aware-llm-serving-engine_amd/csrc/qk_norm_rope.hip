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
// One 512-thread workgroup per token; a 16-lane group per head of the QKV
// row, lane j holding elements 8j..8j+7 (one 16-byte load), so a head's
// statistics are a 16-lane reduction and the RoPE partner of element d
// (d +- 64) sits in lane j ^ 8.  (256-thread workgroups, three heads per
// group at Qwen3-4B's 48 heads, took 10.0 instead of 9.4 us for 1,048
// tokens; one head per group, 768 threads, 9.6 us.)
#include "common.h"
#include "capi_internal.h"

namespace slo {

constexpr int QK_HD = 128;
constexpr int QK_NT = 512;   // threads per workgroup: 32 groups of 16 lanes
constexpr int QK_UNITS = 2;  // heads per 16-lane group: rows of up to 64 heads

// One (token, head) unit: lane j of the 16-lane group holds elements 8j..8j+7
// of head hh in x.  Writes q_out, or k_out and the pool, or the pool.
__device__ __forceinline__ void qk_unit(const u32x4& x, int hh, int j, int64_t tok, int64_t slot, bool store,
                                        int num_heads, int num_kv_heads, const u32x4& wq, const u32x4& wk,
                                        float eps, const float (&c)[8], const float (&s)[8], uint16_t* q_out,
                                        uint16_t* k_out, int kv_dtype, void* k_cache, void* v_cache, float* k_scale,
                                        float* v_scale, float scale_floor) {
#pragma clang fp contract(off)
  const bool is_q = hh < num_heads, is_k = !is_q && hh < num_heads + num_kv_heads;
  const int d0 = 8 * j;
  float f[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_bits_to_f32(x[i] & 0xffffu);
    f[2 * i + 1] = bf16_bits_to_f32(x[i] >> 16);
  }
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
    const u32x4 wv = is_q ? wq : wk;
    // bf16 roundings by v_cvt_pk_bf16_f32 (round to nearest even), two values each.
    float n[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t a = pack_bf16x2(f[2 * i] * r, f[2 * i + 1] * r);
      const uint32_t b = pack_bf16x2(__uint_as_float(a << 16) * bf16_bits_to_f32(wv[i] & 0xffffu),
                                     __uint_as_float(a & 0xffff0000u) * bf16_bits_to_f32(wv[i] >> 16));
      n[2 * i] = __uint_as_float(b << 16);
      n[2 * i + 1] = __uint_as_float(b & 0xffff0000u);
    }
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // element d +- 64: lane j ^ 8 of the 16-lane row (DPP row rotate by 8)
      const float other = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(n[i]), 0x128, 0xf, 0xf, false));
      const float a = n[i] * c[i], b = other * s[i];
      y[i] = j < 8 ? a - b : a + b;  // lanes 0-7: x1 half, lanes 8-15: x2 half
    }
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = pack_bf16x2(y[2 * i], y[2 * i + 1]);
    if (is_q) {
      *reinterpret_cast<u32x4*>(q_out + (tok * num_heads + hh) * QK_HD + d0) = o;
      return;
    }
    *reinterpret_cast<u32x4*>(k_out + (tok * num_kv_heads + kvh) * QK_HD + d0) = o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(o[i] << 16);
      f[2 * i + 1] = __uint_as_float(o[i] & 0xffff0000u);
    }
  }
  if (!store) return;
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

// One workgroup per token: 16-lane group g takes heads g and g+32 of the row
// (all loads first, so a wavefront keeps several in flight).
__global__ void __launch_bounds__(QK_NT)
qk_norm_rope_store_kernel(const uint16_t* __restrict__ qkv, int64_t qkv_stride, const int64_t* __restrict__ positions,
                          int num_heads, int num_kv_heads, const uint16_t* __restrict__ q_w,
                          const uint16_t* __restrict__ k_w, float eps, const float* __restrict__ cos_sin,
                          int max_position, uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_out,
                          const int32_t* __restrict__ slot_mapping, int kv_dtype, void* __restrict__ k_cache,
                          void* __restrict__ v_cache, float* __restrict__ k_scale, float* __restrict__ v_scale,
                          int64_t num_slots, float scale_floor) {
  const int j = threadIdx.x & 15;
  const int grp = threadIdx.x >> 4;
  const int64_t tok = blockIdx.x;
  const int heads = num_heads + 2 * num_kv_heads;
  // Loads in dependency order: the position first (its table row is the only
  // dependent load), then the row's heads and the norm weights.
  int64_t pos = positions[tok];
  const int64_t slot = slot_mapping[tok];
  const uint16_t* row = qkv + tok * qkv_stride + 8 * j;
  u32x4 x[QK_UNITS];
#pragma unroll
  for (int it = 0; it < QK_UNITS; ++it) {
    const int hh = grp + (QK_NT / 16) * it;
    x[it] = hh < heads ? *reinterpret_cast<const u32x4*>(row + (int64_t)hh * QK_HD) : u32x4{0, 0, 0, 0};
  }
  const u32x4 wq = *reinterpret_cast<const u32x4*>(q_w + 8 * j);
  const u32x4 wk = *reinterpret_cast<const u32x4*>(k_w + 8 * j);
  pos = pos < 0 ? 0 : (pos >= max_position ? max_position - 1 : pos);
  const float* cs = cos_sin + pos * QK_HD + ((8 * j) & 63);
  const f32x4 c0 = *reinterpret_cast<const f32x4*>(cs), c1 = *reinterpret_cast<const f32x4*>(cs + 4);
  const f32x4 s0 = *reinterpret_cast<const f32x4*>(cs + 64), s1 = *reinterpret_cast<const f32x4*>(cs + 68);
  const float c[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
  const float s[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
  const bool store = slot >= 0 && slot < num_slots;
#pragma unroll
  for (int it = 0; it < QK_UNITS; ++it) {
    const int hh = grp + (QK_NT / 16) * it;
    if (hh < heads)
      qk_unit(x[it], hh, j, tok, slot, store, num_heads, num_kv_heads, wq, wk, eps, c, s, q_out, k_out, kv_dtype,
              k_cache, v_cache, k_scale, v_scale, scale_floor);
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
  if (num_heads + 2 * num_kv_heads > (QK_NT / 16) * QK_UNITS) return fail(SLO_ERR_UNSUPPORTED, "qk_norm_rope_store: more than 64 heads per row");
  hipLaunchKernelGGL(qk_norm_rope_store_kernel, dim3((unsigned)num_tokens), dim3(QK_NT), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(qkv), qkv_row_stride, positions, num_heads, num_kv_heads,
                     static_cast<const uint16_t*>(q_norm_weight), static_cast<const uint16_t*>(k_norm_weight), eps,
                     cos_sin, max_position, static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_out), slot_mapping,
                     kv_dtype, k_cache, v_cache, k_scale, v_scale, num_slots, scale_floor);
  return check_launch("qk_norm_rope_store");
}
