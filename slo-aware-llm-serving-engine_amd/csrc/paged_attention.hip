// Ragged mixed prefill/decode paged attention for gfx950 (MI355X), one launch.
//
// Replaces the per-phase flash-attn calls of forward_mixed
// (nanovllm/layers/mixed_attention.py:36-57) and of the V0 branches of
// Attention.forward (nanovllm/layers/attention.py:68-78).
//
// Work list.  Every workgroup (4 wavefronts, two workgroups per CU) first
// derives, from the metadata alone, the number of work items of every row and
// their exclusive prefix (prefill rows first, then decode rows), then pulls
// item indices from a device counter (one fetch ahead) until the list is
// exhausted.  The grid is sized from capacities, never from device data, so
// the launch can be recorded in a HIP graph.  The counter and the split-K
// tickets reset themselves at the end of every launch, so no memset is needed.
//
//  * Prefill item (row r, block of 32 query positions, kv head h): each
//    wavefront owns one of the G query heads that share kv head h, for the
//    same positions, so the K/V tiles staged in LDS serve all G heads.  Tiles
//    of 64 keys are double-buffered: the next tile's global loads are in
//    flight while the current one is consumed.  The contraction runs on bf16
//    MFMA (v_mfma_f32_16x16x32_bf16) in the transposed form S^T = K Q^T,
//    O^T += V^T P^T, which keeps each query column's softmax statistics
//    lane-local: the S^T accumulator is the B operand of the PV product
//    without data movement, and V^T comes from the natural [token][d] LDS tile
//    through ds_read_b64_tr_b16.
//  * Decode item (row b, chunk of 256 tokens, kv head h): each wavefront takes
//    64 tokens; the G query heads sharing h are the MFMA columns, K goes from
//    HBM straight into MFMA A-operand registers, V goes from HBM straight into
//    LDS (global_load_lds_dwordx4) for the transposed read.  The 4 wavefronts
//    merge in LDS; a row with several chunks writes one (m, l, acc) partial per
//    chunk and the last chunk to finish merges them (the split-K merge of
//    docs/project_manual.md:643-650).
//
// LDS tiles are 64 rows of 256 bytes with the 16-byte chunks of each row
// XOR-swizzled (K: chunk ^ (row & 15); V: chunk ^ 2*(row & 7)), so the MFMA
// operand reads of 16 lanes fall on distinct banks.
//
// Split-K visibility across XCDs: partials are written and read with
// agent-scope atomic stores/loads (global_store/load ... sc1), which bypass
// the per-XCD L2; each writer waits for its stores to be acknowledged
// (s_waitcnt vmcnt(0)) and the workgroup barrier orders them before the
// ticket increment.  No L2 writeback or invalidate is needed.
//
// Softmax runs in the log2 domain (scores scaled by softmax_scale*log2(e),
// exp2 on v_exp_f32).  Fully-masked tiles never produce exp(-inf - -inf).
//
// FP8 pool: K and V bytes are decoded exactly to bf16 (every E4M3FN value is a
// bf16 value); the per-(token, kv head) K scale multiplies the fp32 score and
// the V scale multiplies the fp32 probability before it is rounded to bf16,
// which is the dequantise-then-attend definition with the scale applied in
// fp32.
#include <algorithm>
#include <mutex>
#include "common.h"
#include "capi_internal.h"

namespace slo {

constexpr int HD = 128;                // head_dim this kernel implements
constexpr int NT = 256;                // threads per workgroup (4 wavefronts)
constexpr int TT = 64;                 // tokens per tile
constexpr int CHUNK = 4 * TT;          // decode split-K chunk
constexpr int ROWB = HD * 2;           // bytes of one bf16 tile row
constexpr int TILE_BYTES = TT * ROWB;  // 16 KiB
constexpr int NQT = 2;                 // 16-position column tiles per prefill wavefront
constexpr int BQ = 16 * NQT;           // query positions per prefill item
constexpr int MAX_ROWS = 1024;         // decode + prefill rows per launch
constexpr int MAX_G = 16;              // query heads per kv head
constexpr int MAX_PAGES = 256;         // prefill block-table entries cached in LDS
constexpr int NLIST = 8;          // work lists (one per XCD)
constexpr int CTRL_STRIDE = 32;   // uint32 words between lists: one 128-byte line each
constexpr int CTRL_BYTES = NLIST * CTRL_STRIDE * 4;
constexpr int MAX_COUNTERS = 65536;
constexpr size_t PARTIALS_OFFSET = CTRL_BYTES + sizeof(int) * (size_t)MAX_COUNTERS;
constexpr float NEG_INF = -__builtin_huge_valf();

struct Params {
  const uint16_t* q;
  int64_t q_stride;
  uint16_t* out;
  int64_t out_stride;
  int32_t num_q_rows;
  const void* k_cache;
  const void* v_cache;
  const float* k_scale;
  const float* v_scale;
  int32_t num_blocks;
  int32_t block_size;
  int32_t nd;             // decode rows taking part in this launch
  int32_t q_off_prefill;  // first query row of prefill row 0
  const int32_t* dlens;
  const int32_t* dtab;
  int32_t dtab_stride;
  int32_t dtab_width;
  int32_t np;
  const int32_t* cu_q;
  const int32_t* cu_k;
  const int32_t* ptab;
  int32_t ptab_stride;
  int32_t ptab_width;
  const uint16_t* k;
  int64_t k_stride;
  const uint16_t* v;
  int64_t v_stride;
  int32_t num_kv_rows;
  int32_t hkv;
  int32_t G;
  int32_t HG;  // ceil(G / 4): wavefront groups per kv head in prefill
  float scale_log2;
  int* ctrl;      // per list: [0] fetch counter, [1] base of the current launch
  int* counters;  // split-K tickets, [num_decode * hkv]
  float* partials;
};

struct Smem {
  union {
    uint8_t dec_v[4][TILE_BYTES];  // decode: one V tile per wavefront
    struct {
      uint8_t k[2][TILE_BYTES];
      uint8_t v[2][TILE_BYTES];
    } pf;                          // prefill: double-buffered K/V tiles
  } u;
  struct {
    float o[4][4][HD];
    float m[4][4];
    float l[4][4];
  } mg;                            // decode: cross-wavefront merge, 4 query heads per pass
  float ks[2][TT];
  float vs[2][TT];
  int pages[MAX_PAGES];  // prefill: block table of the current row
  int off[MAX_ROWS + 1];
  int wsum[4];
  uint32_t item;
  uint32_t base;
  int row;
  int last;
  int salt;
};

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ u32x2 ld8(const void* p) { return *reinterpret_cast<const u32x2*>(p); }
__device__ __forceinline__ void st16(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }

// Byte offset of 16-byte chunk `c` of tile row `r` (K and V swizzles).
__device__ __forceinline__ int k_off(int r, int c) { return r * ROWB + ((c ^ (r & 15)) << 4); }
__device__ __forceinline__ int v_off(int r, int c) { return r * ROWB + ((c ^ ((r & 7) << 1)) << 4); }

__device__ __forceinline__ u32x4 fp8x8_to_bf16x8(const u32x2& w) {
  const u32x2 a = fp8x4_to_bf16x4(w.x), b = fp8x4_to_bf16x4(w.y);
  u32x4 r;
  r.x = a.x;
  r.y = a.y;
  r.z = b.x;
  r.w = b.y;
  return r;
}

__device__ __forceinline__ s16x4 lds_tr16(const uint8_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(const_cast<uint8_t*>(p)));
}

__device__ __forceinline__ bf16x8 join_tr(const s16x4& a, const s16x4& b) {
  const u32x2 x = __builtin_bit_cast(u32x2, a), y = __builtin_bit_cast(u32x2, b);
  u32x4 r;
  r.x = x.x;
  r.y = x.y;
  r.z = y.x;
  r.w = y.y;
  return as_bf16x8(r);
}

// V^T as the A operand of O^T = V^T P^T for k-step `ks` (32 tokens) and
// d-tile `dt`: lane (n, g) receives d = 16dt + n of tokens 32ks + 4g + {0..3}
// (slots 0-3) and 32ks + 16 + 4g + {0..3} (slots 4-7).
__device__ __forceinline__ bf16x8 vt_operand(const uint8_t* tile, int ks, int dt, int g, int n) {
  const int r0 = 32 * ks + 4 * g + (n >> 2);
  const int c = 2 * dt + ((n & 3) >> 1);
  const int half = (n & 1) << 3;
  return join_tr(lds_tr16(tile + v_off(r0, c) + half), lds_tr16(tile + v_off(r0 + 16, c) + half));
}

// max / sum over the 4 lanes {l, l^16, l^32, l^48} (one query column) with
// v_permlane16_swap / v_permlane32_swap instead of LDS-crossbar shuffles.
__device__ __forceinline__ float col_max(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float col_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Online-softmax update of one prefill tile for the wavefront's NQT query
// columns.  Scores stay unscaled until the exponent: max commutes with the
// positive factor c = softmax_scale*log2(e), so e = exp2(c*s - c*m) is one FMA
// and one v_exp_f32 per score.  MASK selects the boundary-tile path (keys past
// the tile's valid rows or causally after the column).
template <bool MASK>
__device__ __forceinline__ void prefill_softmax(f32x4 (&s)[4][NQT], float (&m)[NQT], float (&l)[NQT],
                                                f32x4 (&o)[8][NQT], bf16x8 (&pb)[NQT][2], float c, bool src_fp8,
                                                const float* ks, const float* vs, int g, int ntok, int kv0,
                                                int lim0) {
#pragma unroll
  for (int nt = 0; nt < NQT; ++nt) {
    const int lim = lim0 + 16 * nt;  // last visible key index of this column
    float mx = NEG_INF;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tok = 16 * mt + 4 * g + i;
        float x = s[mt][nt][i];
        if (src_fp8) x *= ks[tok];
        if constexpr (MASK) x = (tok < ntok && kv0 + tok <= lim) ? x : NEG_INF;
        s[mt][nt][i] = x;
        mx = fmaxf(mx, x);
      }
    mx = col_max(mx);
    const float mnew = fmaxf(m[nt], mx);
    const float cm = mnew == NEG_INF ? 0.0f : c * mnew;
    const float alpha = __builtin_amdgcn_exp2f(c * m[nt] - cm);
    float rs = 0.0f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = __builtin_amdgcn_exp2f(fmaf(s[mt][nt][i], c, -cm));
        rs += e;
        s[mt][nt][i] = src_fp8 ? e * vs[16 * mt + 4 * g + i] : e;
      }
    rs = col_sum(rs);
    l[nt] = l[nt] * alpha + rs;
    m[nt] = mnew;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {  // no column's max moved: skip the rescale
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) o[dt][nt] *= alpha;
    }
#pragma unroll
    for (int ks2 = 0; ks2 < 2; ++ks2) {
      u32x4 w;
      w.x = pack_bf16x2(s[2 * ks2][nt][0], s[2 * ks2][nt][1]);
      w.y = pack_bf16x2(s[2 * ks2][nt][2], s[2 * ks2][nt][3]);
      w.z = pack_bf16x2(s[2 * ks2 + 1][nt][0], s[2 * ks2 + 1][nt][1]);
      w.w = pack_bf16x2(s[2 * ks2 + 1][nt][2], s[2 * ks2 + 1][nt][3]);
      pb[nt][ks2] = as_bf16x8(w);
    }
  }
}

__device__ __forceinline__ int decode_len(const Params& p, int b) {
  const int L = p.dlens[b];
  return min(max(L, 0), p.dtab_width * p.block_size);
}

__device__ __forceinline__ int row_items(const Params& p, int r) {
  if (r < p.np) {
    const int lq = p.cu_q[r + 1] - p.cu_q[r];
    return lq > 0 ? ((lq + BQ - 1) / BQ) * p.hkv * p.HG : 0;
  }
  const int L = decode_len(p, r - p.np);
  return max(1, (L + CHUNK - 1) / CHUNK) * p.hkv;
}

__device__ __forceinline__ void store_partial(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_partial(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- decode item
// A decode item is split in three steps so that the next item's HBM loads can
// be in flight while the current item finishes: issue (metadata, Q/K loads to
// registers, V HBM -> LDS), compute (QK, softmax, PV into registers) and tail
// (cross-wavefront merge, split-K partial / ticket / final merge, output).
struct DecodeState {
  int b, h, c, nch, ntok, dindex;
  int64_t slot0;
  u32x4 qv[4];
  u32x4 k[4][4];   // bf16 K operand (bf16 pool)
  u32x2 k8[4][4];  // raw E4M3FN K bytes (E4M3FN pool)
  u32x2 vraw[16];  // raw E4M3FN V rows (bf16 V goes straight to LDS)
  float ksc, vsc;  // E4M3FN scales of token `lane` of this wavefront's tile
};

template <bool FP8>
__device__ __forceinline__ void decode_issue(const Params& p, Smem& sm, DecodeState& st, int b, int local,
                                             int dindex, int tid) {
  const int lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int G = p.G;
  st.b = b;
  st.h = local % p.hkv;
  st.c = local / p.hkv;
  st.dindex = dindex;
  const int L = decode_len(p, b);
  st.nch = max(1, (L + CHUNK - 1) / CHUNK);
  const int t0 = st.c * CHUNK + wave * TT;
  int ntok = min(max(L - t0, 0), TT);
  int64_t slot0 = 0;
  if (ntok > 0) {
    const int page = p.dtab[(int64_t)b * p.dtab_stride + t0 / p.block_size];
    if (page < 0 || page >= p.num_blocks) ntok = 0;  // never dereference padding
    else slot0 = (int64_t)page * p.block_size + (t0 % p.block_size);
  }
  st.ntok = ntok;
  st.slot0 = slot0;
  const int64_t tok_stride = (int64_t)p.hkv * HD;
  const int64_t head_off = (int64_t)st.h * HD;
  uint8_t* vt = sm.u.dec_v[wave];

  // V tile: row r holds token t0 + r; rows past ntok are zeroed.
  if constexpr (!FP8) {
    const uint16_t* vbase = static_cast<const uint16_t*>(p.v_cache) + slot0 * tok_stride + head_off;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = 4 * i + g;  // == lane / 16 within this 4-row stripe
      const int chunk = n ^ ((r & 7) << 1);
      if (r < ntok) __builtin_amdgcn_global_load_lds(vbase + r * tok_stride + 8 * chunk, vt + i * 1024, 16, 0, 0);
      else st16(vt + r * ROWB + (n << 4), u32x4{0, 0, 0, 0});
    }
  } else {
    const uint8_t* vbase = static_cast<const uint8_t*>(p.v_cache) + slot0 * tok_stride + head_off;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = 4 * i + g;
      const int chunk = n ^ ((r & 7) << 1);
      st.vraw[i] = r < ntok ? ld8(vbase + r * tok_stride + 8 * chunk) : u32x2{0, 0};
    }
  }

  // Q as the B operand: column n is query head h*G+n; k slot (g, st, j) is d = 8(4st+g)+j.
  if (n < G) {
    const uint16_t* qr = p.q + (int64_t)b * p.q_stride + (int64_t)(st.h * G + n) * HD;
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) st.qv[s4] = ld16(qr + 8 * (4 * s4 + g));
  } else {
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) st.qv[s4] = u32x4{0, 0, 0, 0};
  }

  // K as the A operand: row (token) 16mt+n, same k slots.
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int tok = 16 * mt + n;
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      const int64_t e = (slot0 + tok) * tok_stride + head_off + 8 * (4 * s4 + g);
      if constexpr (FP8) {
        st.k8[mt][s4] = tok < ntok ? ld8(static_cast<const uint8_t*>(p.k_cache) + e) : u32x2{0, 0};
      } else {
        st.k[mt][s4] = tok < ntok ? ld16(static_cast<const uint16_t*>(p.k_cache) + e) : u32x4{0, 0, 0, 0};
      }
    }
  }

  if constexpr (FP8) {
    const bool ok = lane < ntok;
    const int64_t si = (slot0 + lane) * p.hkv + st.h;
    st.ksc = ok ? p.k_scale[si] : 0.0f;
    st.vsc = ok ? p.v_scale[si] : 0.0f;
  }
}

// QK, softmax and PV of the issued item.  Leaves this wavefront's O^T
// accumulators (lane (n, g): head n, d = 16dt + 4g + i), its max and its sum.
template <bool FP8>
__device__ __forceinline__ void decode_compute(const Params& p, Smem& sm, DecodeState& st, int tid, f32x4 (&o)[8],
                                               float& mx_out, float& ls_out) {
  const int lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int ntok = st.ntok;
  uint8_t* vt = sm.u.dec_v[wave];
  if constexpr (FP8) {
#pragma unroll
    for (int i = 0; i < 16; ++i) st16(vt + (4 * i + g) * ROWB + (n << 4), fp8x8_to_bf16x8(st.vraw[i]));
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) st.k[mt][s4] = fp8x8_to_bf16x8(st.k8[mt][s4]);
  }

  // S^T = K Q^T for the wavefront's 64 tokens.
  f32x4 s[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    s[mt] = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) s[mt] = mfma16(as_bf16x8(st.k[mt][s4]), as_bf16x8(st.qv[s4]), s[mt]);
  }

  float mx = NEG_INF;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tok = 16 * mt + 4 * g + i;
      float x = s[mt][i] * p.scale_log2;
      if constexpr (FP8) x *= __shfl(st.ksc, tok, 64);
      x = tok < ntok ? x : NEG_INF;
      s[mt][i] = x;
      mx = fmaxf(mx, x);
    }
  mx = wave_max_xor(mx, 16);
  mx = wave_max_xor(mx, 32);
  const float mu = mx == NEG_INF ? 0.0f : mx;
  float ls = 0.0f;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float e = __builtin_amdgcn_exp2f(s[mt][i] - mu);
      ls += e;
      if constexpr (FP8) s[mt][i] = e * __shfl(st.vsc, 16 * mt + 4 * g + i, 64);
      else s[mt][i] = e;
    }
  ls += __shfl_xor(ls, 16, 64);
  ls += __shfl_xor(ls, 32, 64);

  // P^T as the B operand of O^T = V^T P^T; k slot (g, j) is token 32ks + 16(j/4) + 4g + j%4.
  bf16x8 pb[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    u32x4 w;
    w.x = pack_bf16x2(s[2 * ks][0], s[2 * ks][1]);
    w.y = pack_bf16x2(s[2 * ks][2], s[2 * ks][3]);
    w.z = pack_bf16x2(s[2 * ks + 1][0], s[2 * ks + 1][1]);
    w.w = pack_bf16x2(s[2 * ks + 1][2], s[2 * ks + 1][3]);
    pb[ks] = as_bf16x8(w);
  }

  // The V tile (LDS DMA, zero rows or decoded E4M3FN rows) must have landed.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = f32x4{0, 0, 0, 0};
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt] = mfma16(vt_operand(vt, ks, dt, g, n), pb[ks], o[dt]);
  mx_out = mx;
  ls_out = ls;
}

// Cross-wavefront merge through LDS, then either the output (single chunk) or
// the split-K partial + ticket, and the final merge by the last chunk.
__device__ __forceinline__ void decode_tail(const Params& p, Smem& sm, int b, int h, int c, int nch, int dindex,
                                            int tid, const f32x4 (&o)[8], float mx, float ls) {
  const int lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int G = p.G;
  float* part = p.partials + (size_t)dindex * G * (HD + 2);
  for (int hg = 0; hg < G; hg += 4) {  // 4 query heads per pass through the merge area
    __syncthreads();
    if (n >= hg && n < min(G, hg + 4)) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) sm.mg.o[wave][n - hg][16 * dt + 4 * g + i] = o[dt][i];
      if (g == 0) {
        sm.mg.m[wave][n - hg] = mx;
        sm.mg.l[wave][n - hg] = ls;
      }
    }
    __syncthreads();
    const int nh = min(4, G - hg);
    for (int idx = tid; idx < nh * HD; idx += NT) {
      const int hl = idx / HD, d = idx % HD, hn = hg + hl;
      float M = NEG_INF;
#pragma unroll
      for (int w = 0; w < 4; ++w) M = fmaxf(M, sm.mg.m[w][hl]);
      float Ls = 0.0f, O = 0.0f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float mw = sm.mg.m[w][hl];
        const float f = mw == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
        Ls += f * sm.mg.l[w][hl];
        O += f * sm.mg.o[w][hl][d];
      }
      if (nch == 1) {
        p.out[(int64_t)b * p.out_stride + (int64_t)(h * G + hn) * HD + d] =
            (uint16_t)f32_to_bf16_bits(Ls > 0.0f ? O / Ls : 0.0f);
      } else {
        store_partial(part + hn * HD + d, O);
        if (d == 0) {
          store_partial(part + G * HD + 2 * hn, M);
          store_partial(part + G * HD + 2 * hn + 1, Ls);
        }
      }
    }
  }
  if (nch == 1) return;

  // Split-K: the last chunk of (row, kv head) to finish merges all partials.
  __builtin_amdgcn_s_waitcnt(0);  // partial stores acknowledged at the coherence point
  __syncthreads();
  if (tid == 0) {
    const int ticket = atomicAdd(&p.counters[b * p.hkv + h], 1);
    sm.last = ticket == nch - 1;
  }
  __syncthreads();
  if (!sm.last) return;
  const int first = dindex - (c * p.hkv + h);
  const size_t pstride = (size_t)p.hkv * G * (HD + 2);  // floats between chunks of one (row, head)
  const float* p0 = p.partials + (size_t)(first + h) * G * (HD + 2);
  for (int idx = tid; idx < G * HD; idx += NT) {
    const int hn = idx / HD, d = idx % HD;
    // One online pass over the chunks; 8 chunks' loads are in flight at a time.
    float M = NEG_INF, Ls = 0.0f, O = 0.0f;
    for (int c0 = 0; c0 < nch; c0 += 8) {
      float mc[8], lc[8], oc[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const bool ok = c0 + u < nch;
        const float* pc = p0 + (size_t)(ok ? c0 + u : c0) * pstride;
        mc[u] = ok ? load_partial(pc + G * HD + 2 * hn) : NEG_INF;
        lc[u] = ok ? load_partial(pc + G * HD + 2 * hn + 1) : 0.0f;
        oc[u] = ok ? load_partial(pc + hn * HD + d) : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float mn = fmaxf(M, mc[u]);
        if (mn == NEG_INF) continue;
        const float a = __builtin_amdgcn_exp2f(M - mn), bw = __builtin_amdgcn_exp2f(mc[u] - mn);
        Ls = Ls * a + lc[u] * bw;
        O = O * a + oc[u] * bw;
        M = mn;
      }
    }
    p.out[(int64_t)b * p.out_stride + (int64_t)(h * G + hn) * HD + d] =
        (uint16_t)f32_to_bf16_bits(Ls > 0.0f ? O / Ls : 0.0f);
  }
  if (tid == 0) atomicExch(&p.counters[b * p.hkv + h], 0);
}

// --------------------------------------------------------------- prefill item
template <bool FP8>
__device__ void prefill_item(const Params& p, Smem& sm, int r, int local, int tid) {
  const int lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int hg = local % p.HG;
  const int t = local / p.HG;
  const int h = t % p.hkv;
  const int qb_rev = t / p.hkv;

  const int q_start = p.cu_q[r];
  const int Lq = p.cu_q[r + 1] - q_start;
  const int k_start = p.cu_k[r];
  const int Lk_full = p.cu_k[r + 1] - k_start;
  const int prefix = Lk_full - Lq;  // bottom-right causal alignment
  const bool paged = p.ptab != nullptr;
  int Lk = Lk_full;
  if (paged) Lk = min(Lk, p.ptab_width * p.block_size);
  else Lk = min(Lk, p.num_kv_rows - k_start);
  Lk = max(Lk, 0);

  const int nqb = (Lq + BQ - 1) / BQ;
  const int q0 = (nqb - 1 - qb_rev) * BQ;  // heaviest blocks are pulled first
  const int qend = min(q0 + BQ, Lq);
  const int kend = min(Lk, max(0, prefix + qend));
  const int hl = hg * 4 + wave;
  const bool active = hl < p.G;
  const int hq = h * p.G + hl;
  const int64_t qrow0 = (int64_t)p.q_off_prefill + q_start;
  const bool src_fp8 = FP8 && paged;

  u32x4 qv[NQT][4];
#pragma unroll
  for (int nt = 0; nt < NQT; ++nt) {
    const int pos = q0 + 16 * nt + n;
    const bool ok = active && pos < Lq && qrow0 + pos < p.num_q_rows;
    const uint16_t* qr = p.q + (qrow0 + pos) * p.q_stride + (int64_t)hq * HD;
#pragma unroll
    for (int st = 0; st < 4; ++st) qv[nt][st] = ok ? ld16(qr + 8 * (4 * st + g)) : u32x4{0, 0, 0, 0};
  }

  f32x4 o[8][NQT];
  float m[NQT], l[NQT];
#pragma unroll
  for (int nt = 0; nt < NQT; ++nt) {
    m[nt] = NEG_INF;
    l[nt] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt][nt] = f32x4{0, 0, 0, 0};
  }

  // Double-buffered tiles: thread covers tile row (tid>>4)+16*it and LDS slot
  // tid&15 of that row (16-byte chunks XOR-swizzled at load time).  bf16
  // sources go HBM -> LDS directly (global_load_lds_dwordx4: lane i of a
  // wavefront lands at byte 16*i of a 1 KiB stripe of 4 rows), so the next
  // tile is in flight while the current one is consumed; E4M3FN pool bytes are
  // loaded into registers, decoded, and written to LDS after the current tile's
  // compute.  Rows past the valid keys are zero.
  u32x4 kr[4], vr[4];
  float ksr = 0.0f, vsr = 0.0f;
  const int* prow = p.ptab + (int64_t)r * p.ptab_stride;
  const int npages = paged ? (kend + p.block_size - 1) / p.block_size : 0;
  const bool cached = npages <= MAX_PAGES;
  typedef __attribute__((address_space(3))) const int lds_int;
  lds_int* pages = (lds_int*)(sm.pages);
  // Lane-constant element offsets of this thread's 4 tile rows (row
  // (tid>>4)+16*it, swizzled 16-byte chunk) from the tile's first key.
  const int krow = paged ? p.hkv * HD : (int)p.k_stride;  // row strides < 2^25 elements (checked on the host)
  const int vrow = paged ? p.hkv * HD : (int)p.v_stride;
  int kgo[4], vgo[4];
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int row = (tid >> 4) + 16 * it;
    kgo[it] = row * krow + 8 * ((tid & 15) ^ (row & 15));
    vgo[it] = row * vrow + 8 * ((tid & 15) ^ ((row & 7) << 1));
  }
  auto issue_tile = [&](int kv0, int buf) {
    const int ntok = min(TT, kend - kv0);
    bool ok = true;
    int64_t slot0 = 0, kbase, vbase;  // element offsets of the tile's first key, head h
    if (paged) {
      const int page = cached ? pages[kv0 / p.block_size] : prow[kv0 / p.block_size];
      ok = page >= 0 && page < p.num_blocks;
      slot0 = ok ? (int64_t)page * p.block_size + kv0 % p.block_size : 0;
      kbase = vbase = slot0 * p.hkv * HD + (int64_t)h * HD;
    } else {
      kbase = (int64_t)(k_start + kv0) * p.k_stride + (int64_t)h * HD;
      vbase = (int64_t)(k_start + kv0) * p.v_stride + (int64_t)h * HD;
    }
    const int nv = ok ? ntok : 0;
    if (src_fp8) {
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int row = (tid >> 4) + 16 * it;
        u32x4 kx = u32x4{0, 0, 0, 0}, vx = u32x4{0, 0, 0, 0};
        if (row < nv) {
          kx = fp8x8_to_bf16x8(ld8(static_cast<const uint8_t*>(p.k_cache) + kbase + kgo[it]));
          vx = fp8x8_to_bf16x8(ld8(static_cast<const uint8_t*>(p.v_cache) + vbase + vgo[it]));
        }
        kr[it] = kx;
        vr[it] = vx;
      }
      if (tid < TT) {
        const bool okt = tid < nv;
        const int64_t si = (slot0 + tid) * p.hkv + h;
        ksr = okt ? p.k_scale[si] : 0.0f;
        vsr = okt ? p.v_scale[si] : 0.0f;
      }
      return;
    }
    const uint16_t* ksrc = (paged ? static_cast<const uint16_t*>(p.k_cache) : p.k) + kbase;
    const uint16_t* vsrc = (paged ? static_cast<const uint16_t*>(p.v_cache) : p.v) + vbase;
    if (nv == TT) {  // full tile: DMA only
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        __builtin_amdgcn_global_load_lds(ksrc + kgo[it], sm.u.pf.k[buf] + (16 * it + 4 * wave) * ROWB, 16, 0, 0);
        __builtin_amdgcn_global_load_lds(vsrc + vgo[it], sm.u.pf.v[buf] + (16 * it + 4 * wave) * ROWB, 16, 0, 0);
      }
      return;
    }
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int row = (tid >> 4) + 16 * it;
      if (row < nv) {
        __builtin_amdgcn_global_load_lds(ksrc + kgo[it], sm.u.pf.k[buf] + (16 * it + 4 * wave) * ROWB, 16, 0, 0);
        __builtin_amdgcn_global_load_lds(vsrc + vgo[it], sm.u.pf.v[buf] + (16 * it + 4 * wave) * ROWB, 16, 0, 0);
      } else {
        st16(sm.u.pf.k[buf] + row * ROWB + ((tid & 15) << 4), u32x4{0, 0, 0, 0});
        st16(sm.u.pf.v[buf] + row * ROWB + ((tid & 15) << 4), u32x4{0, 0, 0, 0});
      }
    }
  };
  auto commit_tile = [&](int buf) {  // register-staged (E4M3FN) tiles only
    if (!src_fp8) return;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int row = (tid >> 4) + 16 * it;
      st16(sm.u.pf.k[buf] + row * ROWB + ((tid & 15) << 4), kr[it]);
      st16(sm.u.pf.v[buf] + row * ROWB + ((tid & 15) << 4), vr[it]);
    }
    if (tid < TT) {
      sm.ks[buf][tid] = ksr;
      sm.vs[buf][tid] = vsr;
    }
  };

  // Lane-constant LDS byte offsets of the MFMA operands within a tile: K rows
  // 16mt+n (mt added per use), V^T rows 32ks + 4g + n/4 (+16 for slots 4-7).
  int koff[4], voff[8];
#pragma unroll
  for (int st = 0; st < 4; ++st) koff[st] = k_off(n, 4 * st + g);
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) voff[dt] = v_off(4 * g + (n >> 2), 2 * dt + ((n & 3) >> 1)) + ((n & 1) << 3);

  // The row's block table goes to LDS once, so no tile waits on a table load.
  if (cached)
    for (int i = tid; i < npages; i += NT) sm.pages[i] = prow[i];
  __syncthreads();
  if (kend > 0) {
    issue_tile(0, 0);
    commit_tile(0);
  }
  for (int kv0 = 0, j = 0; kv0 < kend; kv0 += TT, ++j) {
    const int buf = j & 1;
    const int ntok = min(TT, kend - kv0);
    __builtin_amdgcn_s_waitcnt(0);  // this tile's loads have landed in LDS
    __syncthreads();                // ... for every wavefront; the other buffer is free
    const bool more = kv0 + TT < kend;
    if (more) issue_tile(kv0 + TT, buf ^ 1);
    if (active) {
      const uint8_t* kt = sm.u.pf.k[buf];
      const uint8_t* vt = sm.u.pf.v[buf];

      // S^T = K Q^T; the next K fragment is read while the current one feeds the MFMAs.
      f32x4 s[4][NQT];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < NQT; ++nt) s[mt][nt] = f32x4{0, 0, 0, 0};
      u32x4 kf = ld16(kt + koff[0]);
#pragma unroll
      for (int i = 0; i < 16; ++i) {  // i = 4*mt + st
        const int mt = i >> 2, st = i & 3;
        const u32x4 kn = i + 1 < 16 ? ld16(kt + ((i + 1) >> 2) * 16 * ROWB + koff[(i + 1) & 3]) : kf;
#pragma unroll
        for (int nt = 0; nt < NQT; ++nt) s[mt][nt] = mfma16(as_bf16x8(kf), as_bf16x8(qv[nt][st]), s[mt][nt]);
        kf = kn;
      }

      // Keys that can be masked: beyond the tile's valid rows, or causally
      // after the earliest query column of the block.
      const bool need_mask = ntok < TT || kv0 + TT - 1 > q0 + prefix;
      bf16x8 pb[NQT][2];
      const int lim0 = q0 + n + prefix;
      prefill_softmax<true>(s, m, l, o, pb, p.scale_log2, src_fp8, sm.ks[buf], sm.vs[buf], g, need_mask ? ntok : TT, kv0, need_mask ? lim0 : (1 << 30));

      // O^T += V^T P^T; the next V^T operand is read while the current one feeds the MFMAs.
      auto vload = [&](int i) {
        const uint8_t* va0 = vt + (i >> 3) * 32 * ROWB + voff[i & 7];
        return join_tr(lds_tr16(va0), lds_tr16(va0 + 16 * ROWB));
      };
      bf16x8 va = vload(0);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const bf16x8 vn = i + 1 < 16 ? vload(i + 1) : va;
#pragma unroll
        for (int nt = 0; nt < NQT; ++nt) o[i & 7][nt] = mfma16(va, pb[nt][i >> 3], o[i & 7][nt]);
        va = vn;
      }
    }
    if (more) commit_tile(buf ^ 1);
  }

  if (!active) return;
#pragma unroll
  for (int nt = 0; nt < NQT; ++nt) {
    const int pos = q0 + 16 * nt + n;
    if (pos >= Lq || qrow0 + pos >= p.num_q_rows) continue;
    const float inv = l[nt] > 0.0f ? 1.0f / l[nt] : 0.0f;
    uint16_t* orow = p.out + (qrow0 + pos) * p.out_stride + (int64_t)hq * HD + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      u32x2 w;
      w.x = pack_bf16x2(o[dt][nt][0] * inv, o[dt][nt][1] * inv);
      w.y = pack_bf16x2(o[dt][nt][2] * inv, o[dt][nt][3] * inv);
      *reinterpret_cast<u32x2*>(orow + 16 * dt) = w;
    }
  }
}

// ------------------------------------------------------------------- kernel
template <bool FP8>
__global__ void __launch_bounds__(NT, 2) paged_attention_kernel(Params p) {
  __shared__ Smem sm;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nrows = p.np + p.nd;

  // Per-row item counts -> exclusive prefix in sm.off (block-wide scan).
  const int per = (nrows + NT - 1) / NT;
  const int r0 = tid * per;
  int local_sum = 0;
  for (int r = r0; r < min(r0 + per, nrows); ++r) local_sum += row_items(p, r);
  int incl = local_sum;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(incl, d, 64);
    if (lane >= d) incl += y;
  }
  if (lane == 63) sm.wsum[wave] = incl;
  __syncthreads();
  int run = incl - local_sum;
  for (int w = 0; w < wave; ++w) run += sm.wsum[w];
  for (int r = r0; r < min(r0 + per, nrows); ++r) {
    sm.off[r] = run;
    run += row_items(p, r);
  }
  if (tid == NT - 1) sm.off[nrows] = run;
  __syncthreads();
  const int total = sm.off[nrows];
  const int decode_base = sm.off[p.np];

  // Work lists: item i belongs to list i % nlist and workgroup b serves list
  // b % nlist, so the lists' fetch counters are separate addresses (and, with
  // round-robin dispatch and 8 kv heads, one kv head's prefill tiles stay on
  // one XCD's L2).  A list's counter only grows; the list's base is the
  // counter value at which this launch's items start.  Every workgroup reads
  // the base before its first fetch and stops after its first fetch past the
  // list, so a launch makes exactly count + workgroups fetches on a list and
  // the workgroup that makes the last one advances the base for the next
  // launch.  No counter is ever reset or contended by a completion count.
  const int nlist = min((int)gridDim.x, NLIST);
  const int list = blockIdx.x % nlist;
  const uint32_t count = list < total ? (uint32_t)((total - list + nlist - 1) / nlist) : 0u;
  const uint32_t wgs = (uint32_t)((gridDim.x - list + nlist - 1) / nlist);
  uint32_t* ctr = reinterpret_cast<uint32_t*>(p.ctrl) + list * CTRL_STRIDE;
  if (tid == 0) {
    sm.base = __hip_atomic_load(ctr + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sm.salt = 0;
    sm.item = atomicAdd(ctr, 1u) - sm.base;  // relative fetch index
  }
  __syncthreads();
  const uint32_t base = sm.base;

  // Publishes the fetched-ahead index to the workgroup and returns it.
  auto advance = [&](uint32_t next) -> uint32_t {
    __syncthreads();
    if (tid == 0) sm.item = next;
    __syncthreads();
    return sm.item;
  };
  // Row of relative index `rel`, or -1 past the end of the list.
  auto resolve = [&](uint32_t rel) -> int {
    if (rel >= count) return -1;
    const int item = list + (int)rel * nlist;
    for (int r = tid; r < nrows; r += NT)
      if (sm.off[r] <= item && item < sm.off[r + 1]) sm.row = r;
    __syncthreads();
    return sm.row;
  };

  uint32_t rel = sm.item;
  __syncthreads();
  int r = resolve(rel);
  while (r >= 0) {
    // sm.salt is always 0; reading it here keeps the lane-derived values of the
    // two item paths from being hoisted out of the loop, where they would all
    // stay live at once.
    const int ltid = tid + sm.salt;
    if (r < p.np) {
      const int item = list + (int)rel * nlist;
      uint32_t next = 0;
      if (tid == 0) next = atomicAdd(ctr, 1u) - base;  // fetched ahead, consumed at the end
      prefill_item<FP8>(p, sm, r, item - sm.off[r], ltid);
      rel = advance(next);
      r = resolve(rel);
      continue;
    }
    // A run of decode items: the next item's loads are issued before the
    // current item's merge tail, so HBM stays busy across items.
    DecodeState st;
    {
      const int item = list + (int)rel * nlist;
      decode_issue<FP8>(p, sm, st, r - p.np, item - sm.off[r], item - decode_base, ltid);
    }
    for (;;) {
      uint32_t next = 0;
      if (tid == 0) next = atomicAdd(ctr, 1u) - base;
      f32x4 o[8];
      float mx, ls;
      decode_compute<FP8>(p, sm, st, ltid, o, mx, ls);
      const int cb = st.b, chd = st.h, cc = st.c, cn = st.nch, cdi = st.dindex;
      rel = advance(next);
      r = resolve(rel);
      const bool more = r >= p.np;
      if (more) {
        const int item = list + (int)rel * nlist;
        decode_issue<FP8>(p, sm, st, r - p.np, item - sm.off[r], item - decode_base, ltid);
      }
      decode_tail(p, sm, cb, chd, cc, cn, cdi, ltid, o, mx, ls);
      if (!more) break;
    }
  }
  if (tid == 0 && sm.item == count + wgs - 1u)
    __hip_atomic_store(ctr + 1, base + count + wgs, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct DeviceShape {
  int cus = 0;
  int wg_per_cu[2] = {0, 0};
};

int device_shape(DeviceShape* out) {
  static std::mutex mu;
  static DeviceShape cache[64];
  static bool ready[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return fail(SLO_ERR_HIP, "hipGetDevice failed");
  std::lock_guard<std::mutex> lock(mu);
  if (!ready[dev]) {
    DeviceShape s;
    if (hipDeviceGetAttribute(&s.cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return fail(SLO_ERR_HIP, "hipDeviceGetAttribute failed");
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&s.wg_per_cu[0], paged_attention_kernel<false>, NT, 0) !=
            hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&s.wg_per_cu[1], paged_attention_kernel<true>, NT, 0) !=
            hipSuccess)
      return fail(SLO_ERR_HIP, "occupancy query failed");
    s.wg_per_cu[0] = std::max(1, s.wg_per_cu[0]);
    s.wg_per_cu[1] = std::max(1, s.wg_per_cu[1]);
    cache[dev] = s;
    ready[dev] = true;
  }
  *out = cache[dev];
  return SLO_OK;
}

size_t partial_floats(int64_t items, int G) { return (size_t)items * G * (HD + 2); }

}  // namespace slo

using namespace slo;

extern "C" int slo_attention_workspace_bytes(int32_t max_decode_rows, int32_t max_decode_len, int32_t num_heads,
                                             int32_t num_kv_heads, int32_t head_dim, size_t* bytes) {
  if (!bytes || max_decode_rows < 0 || max_decode_len < 0 || num_kv_heads <= 0 || num_heads <= 0 ||
      num_heads % num_kv_heads)
    return fail(SLO_ERR_INVALID, "workspace_bytes: bad arguments");
  if (head_dim != HD) return fail(SLO_ERR_UNSUPPORTED, "workspace_bytes: head_dim must be 128");
  const int64_t chunks = (max_decode_len + CHUNK - 1) / CHUNK;
  const int64_t items = (int64_t)max_decode_rows * std::max<int64_t>(1, chunks) * num_kv_heads;
  *bytes = PARTIALS_OFFSET + sizeof(float) * partial_floats(items, num_heads / num_kv_heads);
  return SLO_OK;
}

extern "C" int slo_paged_attention(const slo_paged_attention_args* a, slo_stream_t stream) {
  if (!a) return fail(SLO_ERR_INVALID, "paged_attention: null args");
  if (a->head_dim != HD) return fail(SLO_ERR_UNSUPPORTED, "paged_attention: head_dim must be 128");
  if (a->num_kv_heads <= 0 || a->num_heads <= 0 || a->num_heads % a->num_kv_heads)
    return fail(SLO_ERR_INVALID, "paged_attention: num_heads must be a positive multiple of num_kv_heads");
  const int G = a->num_heads / a->num_kv_heads;
  if (G > MAX_G) return fail(SLO_ERR_UNSUPPORTED, "paged_attention: more than 16 query heads per kv head");
  if (a->kv_dtype != KV_BF16 && a->kv_dtype != KV_FP8_E4M3FN) return fail(SLO_ERR_INVALID, "paged_attention: bad kv_dtype");
  const bool do_dec = (a->phases & SLO_PHASE_DECODE) && a->num_decode > 0;
  const bool do_pf = (a->phases & SLO_PHASE_PREFILL) && a->num_prefill > 0;
  if (a->num_decode < 0 || a->num_prefill < 0) return fail(SLO_ERR_INVALID, "paged_attention: negative row count");
  if ((do_dec ? a->num_decode : 0) + (do_pf ? a->num_prefill : 0) > MAX_ROWS)
    return fail(SLO_ERR_UNSUPPORTED, "paged_attention: more than 1024 rows in one launch");
  if (!do_dec && !do_pf) return SLO_OK;
  if (!a->q || !a->out || !a->workspace) return fail(SLO_ERR_INVALID, "paged_attention: null q/out/workspace");
  if ((a->q_row_stride % 8) || (a->out_row_stride % 8) || (reinterpret_cast<uintptr_t>(a->q) % 16) ||
      (reinterpret_cast<uintptr_t>(a->out) % 16))
    return fail(SLO_ERR_INVALID, "paged_attention: q/out rows must be 16-byte aligned");
  const bool fp8 = a->kv_dtype == KV_FP8_E4M3FN;
  const bool need_pool = do_dec || (do_pf && a->prefill_tables);
  if (need_pool) {
    if (!a->k_cache || !a->v_cache || a->num_blocks <= 0) return fail(SLO_ERR_INVALID, "paged_attention: no KV pool");
    if (a->block_size <= 0 || a->block_size % TT)
      return fail(SLO_ERR_UNSUPPORTED, "paged_attention: block_size must be a multiple of 64");
    if (fp8 && (!a->k_scale || !a->v_scale)) return fail(SLO_ERR_INVALID, "paged_attention: FP8 pool needs scales");
  }
  if (do_dec) {
    if (!a->decode_lens || !a->decode_tables || a->decode_table_width <= 0 ||
        a->decode_table_stride < a->decode_table_width)
      return fail(SLO_ERR_INVALID, "paged_attention: bad decode metadata");
    if (a->num_decode > a->num_q_rows) return fail(SLO_ERR_INVALID, "paged_attention: decode rows exceed q rows");
    if ((int64_t)a->num_decode * a->num_kv_heads > MAX_COUNTERS)
      return fail(SLO_ERR_UNSUPPORTED, "paged_attention: too many decode rows x kv heads");
  }
  if (do_pf) {
    if (!a->prefill_cu_q || !a->prefill_cu_k) return fail(SLO_ERR_INVALID, "paged_attention: missing cu_seqlens");
    if (a->prefill_tables) {
      if (a->prefill_table_width <= 0 || a->prefill_table_stride < a->prefill_table_width)
        return fail(SLO_ERR_INVALID, "paged_attention: bad prefill tables");
    } else {
      if (!a->k || !a->v || (a->k_row_stride % 8) || (a->v_row_stride % 8) || a->k_row_stride >= (1 << 25) ||
          a->v_row_stride >= (1 << 25) ||
          (reinterpret_cast<uintptr_t>(a->k) % 16) || (reinterpret_cast<uintptr_t>(a->v) % 16))
        return fail(SLO_ERR_INVALID, "paged_attention: contiguous K/V must be 16-byte aligned bf16 rows");
    }
  }
  // Workspace: control words, split-K tickets, then decode partials.
  size_t need = 0;
  const int dec_len_cap = do_dec ? a->decode_table_width * a->block_size : 0;
  int rc = slo_attention_workspace_bytes(do_dec ? a->num_decode : 0, dec_len_cap, a->num_heads, a->num_kv_heads, HD, &need);
  if (rc) return rc;
  if (a->workspace_bytes < need) return fail(SLO_ERR_WORKSPACE, "paged_attention: workspace too small");
  if (reinterpret_cast<uintptr_t>(a->workspace) % 256) return fail(SLO_ERR_INVALID, "paged_attention: workspace must be 256-byte aligned");

  DeviceShape ds;
  rc = device_shape(&ds);
  if (rc) return rc;

  Params p{};
  p.q = static_cast<const uint16_t*>(a->q);
  p.q_stride = a->q_row_stride;
  p.out = static_cast<uint16_t*>(a->out);
  p.out_stride = a->out_row_stride;
  p.num_q_rows = a->num_q_rows;
  p.k_cache = a->k_cache;
  p.v_cache = a->v_cache;
  p.k_scale = a->k_scale;
  p.v_scale = a->v_scale;
  p.num_blocks = a->num_blocks;
  p.block_size = a->block_size;
  p.nd = do_dec ? a->num_decode : 0;
  p.q_off_prefill = a->num_decode;
  p.dlens = a->decode_lens;
  p.dtab = a->decode_tables;
  p.dtab_stride = a->decode_table_stride;
  p.dtab_width = a->decode_table_width;
  p.np = do_pf ? a->num_prefill : 0;
  p.cu_q = a->prefill_cu_q;
  p.cu_k = a->prefill_cu_k;
  p.ptab = a->prefill_tables;
  p.ptab_stride = a->prefill_table_stride;
  p.ptab_width = a->prefill_table_width;
  p.k = static_cast<const uint16_t*>(a->k);
  p.k_stride = a->k_row_stride;
  p.v = static_cast<const uint16_t*>(a->v);
  p.v_stride = a->v_row_stride;
  p.num_kv_rows = a->num_kv_rows;
  p.hkv = a->num_kv_heads;
  p.G = G;
  p.HG = (G + 3) / 4;
  p.scale_log2 = a->softmax_scale * kLog2e;
  char* ws = static_cast<char*>(a->workspace);
  p.ctrl = reinterpret_cast<int*>(ws);
  p.counters = reinterpret_cast<int*>(ws + CTRL_BYTES);
  p.partials = reinterpret_cast<float*>(ws + PARTIALS_OFFSET);

  // Upper bound on the item count from host-known shapes only.
  int64_t bound = 0;
  if (do_dec) bound += (int64_t)p.nd * ((dec_len_cap + CHUNK - 1) / CHUNK) * p.hkv;
  if (do_pf) {
    const int64_t tq = std::max<int64_t>(0, a->num_q_rows - a->num_decode);
    bound += (tq / BQ + p.np) * p.hkv * p.HG;
  }
  const int64_t slots = (int64_t)ds.cus * ds.wg_per_cu[fp8 ? 1 : 0];
  const int grid = (int)std::max<int64_t>(1, std::min<int64_t>(bound, slots));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (fp8) hipLaunchKernelGGL((paged_attention_kernel<true>), dim3(grid), dim3(NT), 0, s, p);
  else hipLaunchKernelGGL((paged_attention_kernel<false>), dim3(grid), dim3(NT), 0, s, p);
  return check_launch("paged_attention");
}
