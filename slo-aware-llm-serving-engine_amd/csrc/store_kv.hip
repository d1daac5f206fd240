// Slot-mapped KV-cache write with optional E4M3FN quantisation (gfx950).
//
// Replaces the Triton store_kvcache_kernel (nanovllm/layers/attention.py:10-30)
// and implements the quantised store planned in docs/project_manual.md:527-537.
// One workgroup per token; each thread moves one 16-byte chunk (8 bf16) of K or
// V, so a token's num_kv_heads*head_dim row is read and written with fully
// coalesced 16-byte accesses.  In FP8 mode the threads that share a kv head
// (head_dim/8 adjacent lanes of one wavefront) reduce amax with cross-lane
// shuffles and each writes 8 code bytes; the first of them writes the scale.
#include "common.h"
#include "capi_internal.h"

namespace slo {

template <int CPH>  // 16-byte chunks per head = head_dim / 8
__global__ void __launch_bounds__(256)
store_kvcache_kernel(const uint16_t* __restrict__ key, int64_t key_stride,
                     const uint16_t* __restrict__ value, int64_t value_stride,
                     const int32_t* __restrict__ slot_mapping, int32_t num_kv_heads,
                     int32_t kv_dtype, void* __restrict__ k_cache, void* __restrict__ v_cache,
                     float* __restrict__ k_scale, float* __restrict__ v_scale,
                     int64_t num_slots, float scale_floor) {
  const int64_t tok = blockIdx.x;
  const int per = num_kv_heads * CPH;  // chunks per token per tensor
  const int64_t row_elems = (int64_t)num_kv_heads * CPH * 8;
  for (int c = threadIdx.x; c < 2 * per; c += blockDim.x) {
    const bool is_v = c >= per;
    const int cc = is_v ? c - per : c;
    const uint16_t* src = (is_v ? value + tok * value_stride : key + tok * key_stride) + cc * 8;
    // The row's chunk and its slot load together (one round trip); a slot of
    // -1 (a padded row) or past the pool skips the row.
    const u32x4 x = *reinterpret_cast<const u32x4*>(src);
    const int64_t slot = slot_mapping[tok];
    if (slot < 0 || slot >= num_slots) return;
    const int64_t dst = slot * row_elems + (int64_t)cc * 8;
    if (kv_dtype == KV_BF16) {
      uint16_t* cache = static_cast<uint16_t*>(is_v ? v_cache : k_cache);
      *reinterpret_cast<u32x4*>(cache + dst) = x;
    } else {
      float f[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f[2 * j] = bf16_bits_to_f32(x[j] & 0xffffu);
        f[2 * j + 1] = bf16_bits_to_f32(x[j] >> 16);
      }
      float scale;
      const u32x2 packed = e4m3_encode8<CPH>(f, scale_floor, scale);
      uint8_t* cache = static_cast<uint8_t*>(is_v ? v_cache : k_cache);
      *reinterpret_cast<u32x2*>(cache + dst) = packed;
      if ((cc % CPH) == 0) (is_v ? v_scale : k_scale)[slot * num_kv_heads + cc / CPH] = scale;
    }
  }
}

}  // namespace slo

using namespace slo;

extern "C" int slo_store_kvcache(const void* key, int64_t key_row_stride, const void* value,
                                 int64_t value_row_stride, const int32_t* slot_mapping,
                                 int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
                                 int32_t kv_dtype, void* k_cache, void* v_cache, float* k_scale,
                                 float* v_scale, int64_t num_slots, float scale_floor,
                                 slo_stream_t stream) {
  if (num_tokens < 0 || num_kv_heads <= 0) return fail(SLO_ERR_INVALID, "store_kvcache: bad token/head count");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(SLO_ERR_UNSUPPORTED, "store_kvcache: head_dim must be 64, 128 or 256");
  if (kv_dtype != KV_BF16 && kv_dtype != KV_FP8_E4M3FN) return fail(SLO_ERR_INVALID, "store_kvcache: bad kv_dtype");
  if (num_tokens == 0) return SLO_OK;
  if (!key || !value || !slot_mapping || !k_cache || !v_cache) return fail(SLO_ERR_INVALID, "store_kvcache: null pointer");
  if (kv_dtype == KV_FP8_E4M3FN && (!k_scale || !v_scale)) return fail(SLO_ERR_INVALID, "store_kvcache: FP8 needs scale pools");
  if (kv_dtype == KV_FP8_E4M3FN && !(scale_floor > 0.0f)) return fail(SLO_ERR_INVALID, "store_kvcache: scale_floor must be > 0");
  if ((key_row_stride % 8) || (value_row_stride % 8) || (reinterpret_cast<uintptr_t>(key) % 16) ||
      (reinterpret_cast<uintptr_t>(value) % 16) || (reinterpret_cast<uintptr_t>(k_cache) % 16) ||
      (reinterpret_cast<uintptr_t>(v_cache) % 16))
    return fail(SLO_ERR_INVALID, "store_kvcache: rows must be 16-byte aligned (stride multiple of 8 elements)");
  if (2 * num_kv_heads * (head_dim / 8) > 65536) return fail(SLO_ERR_UNSUPPORTED, "store_kvcache: too many heads");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(num_tokens), block(256);
  const auto* k16 = static_cast<const uint16_t*>(key);
  const auto* v16 = static_cast<const uint16_t*>(value);
  switch (head_dim) {
    case 64:
      hipLaunchKernelGGL(store_kvcache_kernel<8>, grid, block, 0, s, k16, key_row_stride, v16, value_row_stride,
                         slot_mapping, num_kv_heads, kv_dtype, k_cache, v_cache, k_scale, v_scale, num_slots, scale_floor);
      break;
    case 128:
      hipLaunchKernelGGL(store_kvcache_kernel<16>, grid, block, 0, s, k16, key_row_stride, v16, value_row_stride,
                         slot_mapping, num_kv_heads, kv_dtype, k_cache, v_cache, k_scale, v_scale, num_slots, scale_floor);
      break;
    default:
      hipLaunchKernelGGL(store_kvcache_kernel<32>, grid, block, 0, s, k16, key_row_stride, v16, value_row_stride,
                         slot_mapping, num_kv_heads, kv_dtype, k_cache, v_cache, k_scale, v_scale, num_slots, scale_floor);
      break;
  }
  return check_launch("store_kvcache");
}
