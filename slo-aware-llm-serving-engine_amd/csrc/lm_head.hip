// LM head on the sampled rows with the greedy argmax fused in (gfx950).
//
// Replaces compute_logits on hidden.index_select(0, sample_indices) and the
// argmax of run_mixed (nanovllm/engine/mixed_model_runner.py:115-126;
// ParallelLMHead.forward, nanovllm/layers/embed_head.py:56-66, at TP=1):
//   logits[r, v] = bf16(sum_k hidden[r, k] * weight[v, k])   (fp32 sums)
//   token[r]     = the first v with the largest logits[r, v]
// The weight (vocab x hidden, 778 MB for Qwen3-4B) is streamed from HBM once;
// the logits need not be written at all.
//
// Workgroup b owns vocab rows [128 b, 128 b + 128): wavefront w the 32 rows
// from 128 b + 32 w, as two 16-row MFMA tiles (v_mfma_f32_16x16x32_bf16, A =
// weight rows, B = hidden^T, so C[vocab][row] leaves every sampled row's
// logits in one lane column).  The hidden rows are staged in LDS 256 or 128
// columns at a time (double-buffered, shared by the 4 wavefronts); each
// wavefront loads the next chunk's weight fragments into registers as soon as
// this chunk's MFMAs have consumed them.  Loads past the last sampled row or
// vocab row repeat the last one, so every lane issues the same loads.  The argmax
// is reduced in registers, across lanes, across wavefronts in LDS, and across
// workgroups with one 64-bit atomicMax per sampled row on the key
// (orderable bf16 bits << 32) | (0xffffffff - v), so the largest value and
// then the smallest index win.  A one-wavefront launch turns the keys into
// token ids and clears them for the next call.
#include "common.h"
#include "capi_internal.h"

namespace slo {

constexpr int LM_RT = 2;            // 16-row weight tiles per wavefront
constexpr int LM_VT = 64 * LM_RT;   // vocab rows per workgroup
// Hidden columns per chunk for NCT row tiles: 256 (each weight row is then
// read 512 contiguous bytes at a time, measured 3% faster than 256 bytes at 26
// sampled rows), halved until the two LDS buffers of the hidden chunk fit in
// 64 KiB (128 from NCT = 3 on).
constexpr int lm_kc(int nct) {
  int kc = 256;
  while (kc > 128 && 2 * nct * 16 * (kc * 2 + 16) > 65536) kc /= 2;
  return kc;
}

__device__ __forceinline__ uint32_t bf16_order(uint32_t b) { return (b & 0x8000u) ? (b ^ 0xffffu) : (b | 0x8000u); }

template <int NCT, int LM_KC = lm_kc(NCT)>  // 16-row tiles of sampled rows, hidden columns per chunk
__global__ void __launch_bounds__(256)
lm_head_argmax_kernel(const uint16_t* __restrict__ hidden, int64_t hstride, int M, const uint16_t* __restrict__ w,
                      int64_t wstride, int V, int H, uint16_t* __restrict__ logits, int64_t lstride,
                      unsigned long long* __restrict__ keys) {
  constexpr int RT = LM_RT;
  constexpr int LM_KS = LM_KC / 32;        // MFMA k-steps per chunk
  constexpr int LM_ROWB = LM_KC * 2 + 16;  // padded LDS row of one hidden chunk (bytes)
  constexpr int HL = NCT * LM_KC / 128;  // 16-byte hidden pieces per thread and chunk
  __shared__ __attribute__((aligned(16))) uint8_t hs[2][NCT * 16 * LM_ROWB];
  __shared__ unsigned long long best[4][NCT * 16];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, n = lane & 15, g = lane >> 4;
  const int vbase = blockIdx.x * LM_VT + wave * 16 * RT;

  // Hidden chunk kc: NCT*16 rows x LM_KC/8 pieces of 16 bytes, spread over the
  // threads, loaded into registers, later written to hs[buf].  Rows past M
  // repeat row M - 1 (their logits are never used), so every lane issues the
  // same loads and the waits stay exact counts.
  auto load_h = [&](int kc, u32x4 (&x)[HL]) {
#pragma unroll
    for (int i = 0; i < HL; ++i) {
      const int c = tid + 256 * i, row = min(c / (LM_KC / 8), M - 1), col = c % (LM_KC / 8);
      x[i] = *reinterpret_cast<const u32x4*>(hidden + row * hstride + kc + 8 * col);
    }
  };
  auto store_h = [&](const u32x4 (&x)[HL], int buf) {
#pragma unroll
    for (int i = 0; i < HL; ++i) {
      const int c = tid + 256 * i;
      *reinterpret_cast<u32x4*>(hs[buf] + (c / (LM_KC / 8)) * LM_ROWB + 16 * (c % (LM_KC / 8))) = x[i];
    }
  };
  // Weight fragments of one chunk: row tile rt, k-step s (32 columns each); a
  // row's LM_KC columns are read by consecutive instructions.
  auto load_a = [&](int kc, u32x4 (&a)[RT][LM_KS]) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int v = vbase + 16 * rt + n;
      const uint16_t* src = w + (int64_t)min(v, V - 1) * wstride + kc + 8 * g;  // rows past V: never ranked
#pragma unroll
      for (int s = 0; s < LM_KS; ++s) a[rt][s] = *reinterpret_cast<const u32x4*>(src + 32 * s);
    }
  };

  f32x4 acc[RT][NCT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) acc[rt][ct] = f32x4{0, 0, 0, 0};

  auto mma = [&](const u32x4 (&cur)[RT][LM_KS], int buf) {
#pragma unroll
    for (int s = 0; s < LM_KS; ++s) {
      u32x4 b[NCT];
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
        b[ct] = *reinterpret_cast<const u32x4*>(hs[buf] + (16 * ct + n) * LM_ROWB + 2 * (32 * s + 8 * g));
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) acc[rt][ct] = mfma16(as_bf16x8(cur[rt][s]), as_bf16x8(b[ct]), acc[rt][ct]);
    }
  };

  const int nchunks = H / LM_KC;
  u32x4 hx[HL];
  // The next chunk's hidden piece is loaded before this chunk's MFMAs and its
  // weight fragments after them, into the same registers (two register sets
  // measured slower: fewer workgroups per CU).
  u32x4 a0[RT][LM_KS];
  load_a(0, a0);
  load_h(0, hx);
  store_h(hx, 0);
  __syncthreads();
  for (int c = 0; c < nchunks; ++c) {
    const int buf = c & 1;
    const bool more = c + 1 < nchunks;
    if (more) load_h((c + 1) * LM_KC, hx);
    mma(a0, buf);
    if (more) {
      load_a((c + 1) * LM_KC, a0);
      store_h(hx, buf ^ 1);
    }
    __syncthreads();
  }

  // Lane (n, g) holds logits of vocab vbase + 16 rt + 4 g + i for sampled row 16 ct + n.
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    const int row = 16 * ct + n;
    unsigned long long key = 0;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int v0 = vbase + 16 * rt + 4 * g;
      const uint32_t p01 = pack_bf16x2(acc[rt][ct][0], acc[rt][ct][1]);
      const uint32_t p23 = pack_bf16x2(acc[rt][ct][2], acc[rt][ct][3]);
      const uint32_t bits[4] = {p01 & 0xffffu, p01 >> 16, p23 & 0xffffu, p23 >> 16};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (v0 + i >= V) continue;
        const unsigned long long k =
            ((unsigned long long)bf16_order(bits[i]) << 32) | (0xffffffffu - (uint32_t)(v0 + i));
        key = k > key ? k : key;
      }
      if (logits != nullptr && row < M && v0 < V) {
        const int64_t off = (int64_t)row * lstride + v0;
        uint16_t* dst = logits + off;
        if (v0 + 3 < V && (off & 3) == 0) {
          *reinterpret_cast<u32x2*>(dst) = u32x2{p01, p23};
        } else {
          for (int i = 0; i < 4 && v0 + i < V; ++i) dst[i] = (uint16_t)bits[i];
        }
      }
    }
#pragma unroll
    for (int m = 16; m < 64; m <<= 1) {
      const unsigned long long o = __shfl_xor(key, m, 64);
      key = o > key ? o : key;
    }
    if (g == 0) best[wave][row] = key;
  }
  __syncthreads();
  for (int row = tid; row < min(M, NCT * 16); row += 256) {
    unsigned long long key = best[0][row];
#pragma unroll
    for (int q = 1; q < 4; ++q) key = best[q][row] > key ? best[q][row] : key;
    if (key) atomicMax(keys + row, key);
  }
}

__global__ void lm_head_tokens_kernel(unsigned long long* __restrict__ keys, int64_t* __restrict__ tokens, int M) {
  for (int r = threadIdx.x; r < M; r += blockDim.x) {
    const unsigned long long k = keys[r];
    tokens[r] = (int64_t)(0xffffffffu - (uint32_t)(k & 0xffffffffu));
    keys[r] = 0;
  }
}

template <int NCT>
void launch_lm(dim3 grid, hipStream_t s, const uint16_t* hidden, int64_t hstride, int M, const uint16_t* w,
               int64_t wstride, int V, int H, uint16_t* logits, int64_t lstride, unsigned long long* keys) {
  if (H % lm_kc(NCT) == 0)
    hipLaunchKernelGGL((lm_head_argmax_kernel<NCT, lm_kc(NCT)>), grid, dim3(256), 0, s, hidden, hstride, M, w, wstride, V,
                       H, logits, lstride, keys);
  else
    hipLaunchKernelGGL((lm_head_argmax_kernel<NCT, 128>), grid, dim3(256), 0, s, hidden, hstride, M, w, wstride, V, H,
                       logits, lstride, keys);
}

}  // namespace slo

using namespace slo;

extern "C" int slo_lm_head_argmax(const void* hidden, int64_t hidden_row_stride, int32_t num_rows, const void* weight,
                                  int64_t weight_row_stride, int32_t vocab_size, int32_t hidden_size, void* logits,
                                  int64_t logits_row_stride, uint64_t* keys, int64_t* tokens, slo_stream_t stream) {
  if (num_rows < 0 || vocab_size <= 0 || hidden_size <= 0) return fail(SLO_ERR_INVALID, "lm_head_argmax: bad sizes");
  if (num_rows > 128) return fail(SLO_ERR_UNSUPPORTED, "lm_head_argmax: at most 128 sampled rows per call");
  if (hidden_size % 128) return fail(SLO_ERR_UNSUPPORTED, "lm_head_argmax: hidden_size must be a multiple of 128");
  if (num_rows == 0) return SLO_OK;
  if (!hidden || !weight || !keys || !tokens) return fail(SLO_ERR_INVALID, "lm_head_argmax: null pointer");
  if ((hidden_row_stride % 8) || (weight_row_stride % 8) || hidden_row_stride < hidden_size ||
      weight_row_stride < hidden_size || (reinterpret_cast<uintptr_t>(hidden) % 16) ||
      (reinterpret_cast<uintptr_t>(weight) % 16) || (reinterpret_cast<uintptr_t>(keys) % 8))
    return fail(SLO_ERR_INVALID, "lm_head_argmax: rows must be 16-byte aligned");
  if (logits && (logits_row_stride < vocab_size || (reinterpret_cast<uintptr_t>(logits) % 8)))
    return fail(SLO_ERR_INVALID, "lm_head_argmax: logits must be 8-byte aligned with rows of at least vocab_size");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((vocab_size + LM_VT - 1) / LM_VT);
  const auto* h16 = static_cast<const uint16_t*>(hidden);
  const auto* w16 = static_cast<const uint16_t*>(weight);
  auto* l16 = static_cast<uint16_t*>(logits);
  auto* k64 = reinterpret_cast<unsigned long long*>(keys);
  switch ((num_rows + 15) / 16) {
    case 1: launch_lm<1>(grid, s, h16, hidden_row_stride, num_rows, w16, weight_row_stride, vocab_size, hidden_size, l16, logits_row_stride, k64); break;
    case 2: launch_lm<2>(grid, s, h16, hidden_row_stride, num_rows, w16, weight_row_stride, vocab_size, hidden_size, l16, logits_row_stride, k64); break;
    case 3: launch_lm<3>(grid, s, h16, hidden_row_stride, num_rows, w16, weight_row_stride, vocab_size, hidden_size, l16, logits_row_stride, k64); break;
    case 4: launch_lm<4>(grid, s, h16, hidden_row_stride, num_rows, w16, weight_row_stride, vocab_size, hidden_size, l16, logits_row_stride, k64); break;
    case 5: launch_lm<5>(grid, s, h16, hidden_row_stride, num_rows, w16, weight_row_stride, vocab_size, hidden_size, l16, logits_row_stride, k64); break;
    case 6: launch_lm<6>(grid, s, h16, hidden_row_stride, num_rows, w16, weight_row_stride, vocab_size, hidden_size, l16, logits_row_stride, k64); break;
    case 7: launch_lm<7>(grid, s, h16, hidden_row_stride, num_rows, w16, weight_row_stride, vocab_size, hidden_size, l16, logits_row_stride, k64); break;
    default: launch_lm<8>(grid, s, h16, hidden_row_stride, num_rows, w16, weight_row_stride, vocab_size, hidden_size, l16, logits_row_stride, k64); break;
  }
  int rc = check_launch("lm_head_argmax");
  if (rc) return rc;
  hipLaunchKernelGGL(lm_head_tokens_kernel, dim3(1), dim3(128), 0, s, k64, tokens, num_rows);
  return check_launch("lm_head_tokens");
}
