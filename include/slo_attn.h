/*
 * slo_attn.h -- C-ABI of the MI355X (gfx950) attention hot path for the
 * SLO-aware nano-vLLM engine.
 *
 * All pointers are raw device pointers owned by the caller (PyTorch tensors in
 * the Python host layer).  All entry points are asynchronous on `stream`
 * (a hipStream_t), never synchronise the device, never allocate device memory
 * and never abort: they return SLO_OK or an error code, and slo_last_error()
 * describes the last failure on the calling thread.  Every launch has a grid
 * sized from shapes and capacities only, so calls may be recorded into a HIP
 * graph.
 *
 * Pool geometry (per layer), identical to the reference engine:
 *   K/V   [num_blocks, block_size, num_kv_heads, head_dim]  bf16, or E4M3FN
 *         bytes when kv_dtype == SLO_KV_FP8_E4M3FN
 *   scale [num_blocks, block_size, num_kv_heads]            fp32 (FP8 only)
 *   slot  = block_table[pos / block_size] * block_size + pos % block_size
 */
#ifndef SLO_ATTN_H_
#define SLO_ATTN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* slo_stream_t; /* hipStream_t */

enum {
  SLO_OK = 0,
  SLO_ERR_INVALID = 1,     /* bad argument, shape or stride */
  SLO_ERR_HIP = 2,         /* a HIP runtime call failed */
  SLO_ERR_WORKSPACE = 3,   /* workspace smaller than slo_attention_workspace_bytes */
  SLO_ERR_UNSUPPORTED = 4, /* geometry this build does not implement */
  SLO_ERR_STATE = 5        /* a workspace word that must be zero between launches is not */
};

enum { SLO_KV_BF16 = 0, SLO_KV_FP8_E4M3FN = 1 };

enum { SLO_PHASE_DECODE = 1, SLO_PHASE_PREFILL = 2, SLO_PHASE_ALL = 3 };

/* Smallest FP8 scale: a power of two, so a scale is always a normal fp32 and
 * no denormal arithmetic can change a code. */
#define SLO_FP8_SCALE_FLOOR 5.421010862427522e-20f /* 2^-64 */

/*
 * Slot-mapped KV-cache write, optionally quantising to E4M3FN.
 *
 * Replaces store_kvcache / store_kvcache_kernel
 * (nanovllm/layers/attention.py:10-40): for every token i with
 * slot_mapping[i] != -1, row i of key/value (num_kv_heads*head_dim contiguous
 * elements, rows `key_row_stride` / `value_row_stride` elements apart) is
 * written to slot slot_mapping[i] of k_cache / v_cache.  With
 * kv_dtype == SLO_KV_FP8_E4M3FN it implements the store of the quantised pool
 * specified in docs/project_manual.md:527-537,583: per (token, kv head)
 *   amax = max|x|; scale = amax == 0 ? 1 : max(amax / 448, scale_floor)
 *   code = E4M3FN_RNE(clamp(x / scale, -448, 448)); k_scale[slot, head] = scale
 * key/value are bf16.  Slots outside [0, num_slots) are skipped like -1.
 */
int slo_store_kvcache(const void* key, int64_t key_row_stride,
                      const void* value, int64_t value_row_stride,
                      const int32_t* slot_mapping, int32_t num_tokens,
                      int32_t num_kv_heads, int32_t head_dim, int32_t kv_dtype,
                      void* k_cache, void* v_cache, float* k_scale, float* v_scale,
                      int64_t num_slots, float scale_floor, slo_stream_t stream);

/*
 * Fused q/k RMSNorm, rotary embedding and KV-cache write, one pass over the
 * fused QKV projection output.
 *
 * Replaces the steps between qkv_proj and the attention call in
 * Qwen3Attention.forward (nanovllm/models/qwen3.py:80-86): q_norm and k_norm
 * (RMSNorm over head_dim, nanovllm/layers/layernorm.py:16-26), rotary_emb
 * (nanovllm/layers/rotary_embedding.py:6-14,37-48) and the store_kvcache that
 * Attention.forward issues before attending (nanovllm/layers/attention.py:
 * 10-40,59-66).  Row i of `qkv` holds num_heads q heads, then num_kv_heads k
 * heads, then num_kv_heads v heads of head_dim bf16 each (rows
 * `qkv_row_stride` elements apart).  Writes q_out [num_tokens, num_heads,
 * head_dim] and k_out [num_tokens, num_kv_heads, head_dim] (bf16, contiguous;
 * q and k normalised and rotated), and, for tokens whose slot is not -1, the
 * rotated k and the unchanged v into the pool exactly as slo_store_kvcache
 * does (E4M3FN with scales when kv_dtype says so).  positions are int64;
 * cos_sin is the fp32 [max_position, head_dim] table whose row p is
 * cos(p*inv_freq) then sin(p*inv_freq) (the reference's cos_sin_cache);
 * positions outside [0, max_position) are clamped into it.  q/k norm weights
 * are bf16 [head_dim].  head_dim must be 128.
 */
int slo_qk_norm_rope_store(const void* qkv, int64_t qkv_row_stride, const int64_t* positions,
                           int32_t num_tokens, int32_t num_heads, int32_t num_kv_heads,
                           int32_t head_dim, const void* q_norm_weight, const void* k_norm_weight,
                           float eps, const float* cos_sin, int32_t max_position, void* q_out,
                           void* k_out, const int32_t* slot_mapping, int32_t kv_dtype,
                           void* k_cache, void* v_cache, float* k_scale, float* v_scale,
                           int64_t num_slots, float scale_floor, slo_stream_t stream);

/*
 * LM head on the sampled rows with the greedy argmax fused in.
 *
 * Replaces compute_logits on the sampled hidden rows and the greedy argmax of
 * run_mixed (nanovllm/engine/mixed_model_runner.py:115-126; ParallelLMHead,
 * nanovllm/layers/embed_head.py:56-66, at TP=1): for each of num_rows rows of
 * `hidden` (bf16, rows `hidden_row_stride` apart), logits[r, v] =
 * bf16(sum_k hidden[r, k] * weight[v, k]) with fp32 sums over the bf16
 * `weight` [vocab_size, hidden_size] (rows `weight_row_stride` apart), and
 * tokens[r] (int64) = the first v with the largest logits[r, v].  `logits`
 * [num_rows, >= vocab_size] bf16 is written only when not NULL.  `keys` is a
 * uint64 [num_rows] scratch array that must be zero before the first call;
 * every call leaves it zero.  num_rows <= 128; hidden_size a multiple of 128.
 */
int slo_lm_head_argmax(const void* hidden, int64_t hidden_row_stride, int32_t num_rows,
                       const void* weight, int64_t weight_row_stride, int32_t vocab_size,
                       int32_t hidden_size, void* logits, int64_t logits_row_stride,
                       uint64_t* keys, int64_t* tokens, slo_stream_t stream);

/*
 * Mixed-step metadata on the GPU, capacity-padded for graph replay.
 *
 * Replaces the host loops of build_batch (nanovllm/engine/batch_metadata.py:
 * 94-118) and prepare_mixed (nanovllm/engine/mixed_model_runner.py:58-92).
 * Rows [0, decode_capacity) are decode rows (row_tokens 1, or 0 for an unused
 * row), rows [decode_capacity, decode_capacity + prefill_capacity) prefill
 * rows (row_tokens >= 0); row_start is each row's first new position and
 * tables its block table ([rows, >= table_width], -1 padded).  Token b is
 * decode row b; token decode_capacity + cu_seqlens_q[r] + i is token i of
 * prefill row r.  Writes positions (int64) and slot_mapping for
 * token_capacity tokens (slot -1, position 0 past the rows' tokens),
 * decode_lens (end_pos, 0 for unused rows), cu_seqlens_q / cu_seqlens_k
 * [prefill_capacity + 1] (sums of num_tokens / end_pos) and last_token
 * [decode_capacity + prefill_capacity] (-1 for rows without tokens).  At most
 * 1024 prefill rows.
 */
int slo_build_mixed_metadata(const int32_t* row_start, const int32_t* row_tokens,
                             int32_t decode_capacity, int32_t prefill_capacity,
                             int32_t token_capacity, const int32_t* tables, int32_t table_stride,
                             int32_t table_width, int32_t block_size, int64_t* positions,
                             int32_t* slot_mapping, int32_t* decode_lens, int32_t* cu_seqlens_q,
                             int32_t* cu_seqlens_k, int32_t* last_token, slo_stream_t stream);

/*
 * Arguments of one ragged paged-attention launch.  Query rows [0, num_decode)
 * are decode rows (one query each, attending to decode_lens[b] cached tokens
 * through decode_tables[b]); query rows num_decode + [cu_q[r], cu_q[r+1]) are
 * the queries of prefill row r, attending causally (bottom-right aligned:
 * key j is visible to query i iff j <= i + Lk - Lq) to Lk = cu_k[r+1]-cu_k[r]
 * keys read from the pool through prefill_tables[r], or, when
 * prefill_tables is NULL, from the contiguous new K/V rows k/v starting at
 * row cu_k[r].  GQA maps query head h to kv head h / (num_heads/num_kv_heads).
 */
typedef struct slo_paged_attention_args {
  const void* q;              /* bf16 [num_q_rows, num_heads, head_dim] */
  int64_t q_row_stride;       /* elements between query rows */
  void* out;                  /* bf16 [num_q_rows, num_heads, head_dim] */
  int64_t out_row_stride;
  int32_t num_q_rows;

  const void* k_cache;        /* pool, see file comment */
  const void* v_cache;
  const float* k_scale;       /* FP8 only, else NULL */
  const float* v_scale;
  int32_t kv_dtype;
  int32_t num_blocks;
  int32_t block_size;         /* multiple of 64 */

  int32_t num_decode;
  const int32_t* decode_lens;     /* [num_decode] */
  const int32_t* decode_tables;   /* [num_decode, >= decode_table_width], -1 padded */
  int32_t decode_table_stride;
  int32_t decode_table_width;

  int32_t num_prefill;
  const int32_t* prefill_cu_q;    /* [num_prefill + 1] */
  const int32_t* prefill_cu_k;    /* [num_prefill + 1] */
  int32_t max_q;                  /* host bounds: max over rows of Lq and Lk */
  int32_t max_k;
  const int32_t* prefill_tables;  /* [num_prefill, >= width] or NULL */
  int32_t prefill_table_stride;
  int32_t prefill_table_width;
  const void* k;                  /* contiguous bf16 K/V, used iff prefill_tables == NULL */
  int64_t k_row_stride;           /* elements, >= num_kv_heads * 128 */
  const void* v;
  int64_t v_row_stride;
  int32_t num_kv_rows;

  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t head_dim;               /* 128 */
  float softmax_scale;

  void* workspace;                /* zero-filled once at allocation */
  size_t workspace_bytes;
  int32_t phases;                 /* SLO_PHASE_* mask */

  /* Optional KV write in the same launch, the store of
   * forward_mixed / Attention.forward (nanovllm/layers/mixed_attention.py:
   * 33, nanovllm/layers/attention.py:66-67) folded into the attention
   * launch (with an E4M3FN pool: the quantising store of
   * slo_store_kvcache with store_scale_floor, and at most 8 query heads per
   * kv head).  When store_slot_mapping is not NULL, new row t of new_k/new_v
   * ([num_new_rows == num_q_rows, num_kv_heads, head_dim] bf16, contiguous:
   * row stride num_kv_heads * head_dim, 16-byte aligned; decode rows' tokens first,
   * then the prefill rows' tokens in cu_seqlens_q order) is written to pool
   * slot store_slot_mapping[t] (slots < 0 or past the pool are skipped), and
   * the launch reads the step's new tokens from new_k/new_v instead of the
   * pool: token decode_lens[b] - 1 of decode row b is new row b, and key j >=
   * Lk - Lq of a prefill row read through prefill_tables is new row
   * num_decode + cu_q[r] + j - (Lk - Lq).  The result equals the separate
   * store followed by this launch, bit for bit; no slot written by the launch
   * may be read through a table by it except as such a new token.  Launches
   * without decode rows, and E4M3FN launches with prefill rows, make that
   * order themselves: the store kernel, then the attention launch (two
   * kernels on `stream`, the same bytes and outputs). */
  const int32_t* store_slot_mapping;  /* [num_new_rows] or NULL */
  const void* new_k;
  int64_t new_k_row_stride;
  const void* new_v;
  int64_t new_v_row_stride;
  int32_t num_new_rows;
  float store_scale_floor;  /* E4M3FN pools: scale_floor of the folded store (> 0) */
} slo_paged_attention_args;

/*
 * Bytes of workspace one launch needs when at most `max_decode_rows` decode
 * rows of at most `max_decode_len` tokens each are present.
 */
int slo_attention_workspace_bytes(int32_t max_decode_rows, int32_t max_decode_len,
                                  int32_t num_heads, int32_t num_kv_heads,
                                  int32_t head_dim, size_t* bytes);

/*
 * One launch of the ragged mixed prefill/decode paged attention.
 *
 * Replaces, in one kernel, the per-phase flash-attn calls of forward_mixed
 * (nanovllm/layers/mixed_attention.py:36-57: flash_attn_with_kvcache on rows
 * [:d], flash_attn_varlen_func on rows [d:], torch.cat), the V0 decode call
 * (nanovllm/layers/attention.py:75-78) and the V0 prefill call
 * (nanovllm/layers/attention.py:68-74).  The work list (split-K decode chunks
 * and prefill query tiles) is built on the GPU from the metadata, and split-K
 * partials are merged inside the same launch.  The grid is the number of
 * workgroups of the launched kernel the GPU holds at once, so a merge's chunks
 * are computed while it waits; should they not arrive within the bounded wait
 * (see slo_attention_workspace_check) the merge gives up and the event is
 * counted.  Every work-list counter and ticket of the workspace is zero again
 * when the launch ends.  Launches that share one workspace must be ordered on
 * one stream.
 */
int slo_paged_attention(const slo_paged_attention_args* args, slo_stream_t stream);

/*
 * Diagnostic, not for the hot path: waits for `stream`, then checks the state
 * every slo_paged_attention launch leaves in `workspace`: every work-list
 * counter and split-K ticket zero, and no split-K merge that gave up waiting.
 * (A merge task waits at most 200 ms, or SLO_ATTN_MERGE_WAIT_US microseconds,
 * for the chunks of its (row, kv head); chunks come from workgroups of the same
 * launch, which are all resident unless another kernel holds the GPU's compute
 * units.  A task that gives up writes nothing for its rows and counts the
 * event; the tickets still return to zero, so later launches are unaffected.)
 * Returns SLO_OK, or SLO_ERR_STATE naming a nonzero word (the workspace must
 * then be zero-filled before its next launch) or the number of merges that
 * gave up since the last check (their decode outputs are invalid).  When
 * `events` is not NULL it receives the 4 event counters, [0] merges that gave
 * up, [1] split prefill item pairs merged, [2..3] zero; the counters are
 * cleared, so each event is reported once.  With workspace NULL and
 * workspace_bytes 0 it checks the static scratch of slo_paged_attention_noalloc
 * on the current device.  It synchronises, so it refuses a stream under
 * capture.  No counterpart in the reference (flash-attn keeps no
 * state between calls): it backs the contract of slo_paged_attention.
 */
int slo_attention_workspace_check(const void* workspace, size_t workspace_bytes, uint32_t* events,
                                  slo_stream_t stream);

/*
 * slo_paged_attention without a caller workspace, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference (its
 * flash-attn calls allocate their own outputs).  Same arguments and results as
 * slo_paged_attention except that args->workspace must be NULL and
 * args->workspace_bytes 0: the launch uses the library's static device array
 * of SLO_NOALLOC_SCRATCH_BYTES per GPU (zero at load, held until the process
 * ends; its address is looked up once per device), and calls nothing that
 * allocates.  A launch whose decode rows need more split-K partials than the
 * array holds after its 260 KiB control area (rows x ceil(table width x
 * block_size / 128) x num_heads x 528 bytes) is refused with
 * SLO_ERR_UNSUPPORTED.  Every call on one GPU shares its array, so calls that
 * overlap on one GPU (several streams, several threads) race; order them on
 * one stream.  slo_attention_workspace_check(NULL, 0, ...) checks this array
 * on the current device.
 */
#define SLO_NOALLOC_SCRATCH_BYTES (64u << 20)
int slo_paged_attention_noalloc(const slo_paged_attention_args* args, slo_stream_t stream);

/* Description of the last error on the calling thread ("" if none). */
const char* slo_last_error(void);

/* Size of slo_paged_attention_args, for binding checks. */
size_t slo_paged_attention_args_size(void);

#ifdef __cplusplus
}
#endif

#endif /* SLO_ATTN_H_ */
