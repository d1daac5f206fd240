// Mixed-step attention metadata built on the GPU, in a capacity-padded layout
// that a captured HIP graph can replay for any batch that fits (gfx950).
//
// Replaces the host-side loops of build_batch (nanovllm/engine/
// batch_metadata.py:94-118) and prepare_mixed (nanovllm/engine/
// mixed_model_runner.py:58-92), which build positions, slot_mapping,
// decode_lens, cu_seqlens_q/k and the sample indices in Python and copy each
// to the device.  Here the host sends one (start_pos, num_tokens) pair per row
// and the rows' block tables; one workgroup derives the rest:
//   rows [0, Dc)        decode rows: 1 token (0 = unused slot of the capacity)
//   rows [Dc, Dc + Pc)  prefill rows: num_tokens >= 0 new tokens
//   token b             decode row b (position start_pos)
//   token Dc + cu_q[r] + i   token i of prefill row r (position start_pos + i)
//   slot = table[row][pos / block_size] * block_size + pos % block_size
//   decode_lens[b] = start_pos + 1 (end_pos), 0 for an unused row
//   cu_q / cu_k = prefix sums of num_tokens / end_pos over prefill rows (0
//   for a row without tokens), last_token[row] = index of its last token
// Tokens not covered by a row get slot -1 and position 0, so the store kernels
// skip them and attention never reads them.
#include "common.h"
#include "capi_internal.h"

namespace slo {

constexpr int MD_NT = 1024;
constexpr int MD_MAX_PF = 1024;

__global__ void __launch_bounds__(MD_NT)
mixed_metadata_kernel(const int32_t* __restrict__ row_start, const int32_t* __restrict__ row_tokens, int Dc, int Pc,
                      int token_cap, const int32_t* __restrict__ tables, int table_stride, int table_width,
                      int block_size, int64_t* __restrict__ positions, int32_t* __restrict__ slot_mapping,
                      int32_t* __restrict__ decode_lens, int32_t* __restrict__ cu_q, int32_t* __restrict__ cu_k,
                      int32_t* __restrict__ last_token) {
  __shared__ int q_off[MD_MAX_PF + 1];
  __shared__ int wsum[2][MD_NT / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  auto slot_of = [&](int row, int pos) -> int32_t {
    const int page_idx = pos / block_size;
    if (pos < 0 || page_idx >= table_width) return -1;
    const int page = tables[(int64_t)row * table_stride + page_idx];
    return page < 0 ? -1 : page * block_size + pos % block_size;
  };

  // Prefill rows: exclusive prefix sums of tokens and of end_pos.
  int nq = 0, nk = 0;
  if (tid < Pc) {
    nq = max(row_tokens[Dc + tid], 0);
    nk = nq > 0 ? row_start[Dc + tid] + nq : 0;
  }
  int iq = nq, ik = nk;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int yq = __shfl_up(iq, d, 64), yk = __shfl_up(ik, d, 64);
    if (lane >= d) {
      iq += yq;
      ik += yk;
    }
  }
  if (lane == 63) {
    wsum[0][wave] = iq;
    wsum[1][wave] = ik;
  }
  __syncthreads();
  int bq = 0, bk = 0;
  for (int w = 0; w < wave; ++w) {
    bq += wsum[0][w];
    bk += wsum[1][w];
  }
  if (tid < Pc) {
    q_off[tid] = bq + iq - nq;
    cu_q[tid] = bq + iq - nq;
    cu_k[tid] = bk + ik - nk;
    last_token[Dc + tid] = nq > 0 ? Dc + bq + iq - 1 : -1;
  }
  if (tid == Pc - 1 || (Pc == 0 && tid == 0)) {
    q_off[Pc] = Pc ? bq + iq : 0;
    cu_q[Pc] = Pc ? bq + iq : 0;
    cu_k[Pc] = Pc ? bk + ik : 0;
  }
  __syncthreads();

  // Decode rows: one token each.
  for (int b = tid; b < Dc; b += MD_NT) {
    const bool live = row_tokens[b] > 0 && b < token_cap;
    const int pos = row_start[b];
    if (b < token_cap) {
      positions[b] = live ? pos : 0;
      slot_mapping[b] = live ? slot_of(b, pos) : -1;
    }
    decode_lens[b] = live ? pos + 1 : 0;
    last_token[b] = live ? b : -1;
  }
  // Prefill tokens and the padding after them.
  const int total = q_off[Pc];
  for (int t = Dc + tid; t < token_cap; t += MD_NT) {
    const int rel = t - Dc;
    if (rel >= total) {
      positions[t] = 0;
      slot_mapping[t] = -1;
      continue;
    }
    int lo = 0, hi = Pc;  // largest r with q_off[r] <= rel
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (q_off[mid] <= rel) lo = mid;
      else hi = mid;
    }
    const int pos = row_start[Dc + lo] + (rel - q_off[lo]);
    positions[t] = pos;
    slot_mapping[t] = slot_of(Dc + lo, pos);
  }
}

}  // namespace slo

using namespace slo;

extern "C" int slo_build_mixed_metadata(const int32_t* row_start, const int32_t* row_tokens, int32_t decode_capacity,
                                        int32_t prefill_capacity, int32_t token_capacity, const int32_t* tables,
                                        int32_t table_stride, int32_t table_width, int32_t block_size,
                                        int64_t* positions, int32_t* slot_mapping, int32_t* decode_lens,
                                        int32_t* cu_seqlens_q, int32_t* cu_seqlens_k, int32_t* last_token,
                                        slo_stream_t stream) {
  if (decode_capacity < 0 || prefill_capacity < 0 || token_capacity < 0 || table_width <= 0 ||
      table_stride < table_width || block_size <= 0)
    return fail(SLO_ERR_INVALID, "build_mixed_metadata: bad sizes");
  if (prefill_capacity > MD_MAX_PF)
    return fail(SLO_ERR_UNSUPPORTED, "build_mixed_metadata: more than 1024 prefill rows");
  if (token_capacity < decode_capacity)
    return fail(SLO_ERR_INVALID, "build_mixed_metadata: token capacity below the decode rows");
  if (!row_start || !row_tokens || !tables || !positions || !slot_mapping || !cu_seqlens_q || !cu_seqlens_k ||
      !last_token || (decode_capacity && !decode_lens))
    return fail(SLO_ERR_INVALID, "build_mixed_metadata: null pointer");
  hipLaunchKernelGGL(mixed_metadata_kernel, dim3(1), dim3(MD_NT), 0, static_cast<hipStream_t>(stream), row_start,
                     row_tokens, decode_capacity, prefill_capacity, token_capacity, tables, table_stride, table_width,
                     block_size, positions, slot_mapping, decode_lens, cu_seqlens_q, cu_seqlens_k, last_token);
  return check_launch("build_mixed_metadata");
}
