// Ragged mixed prefill/decode paged attention for gfx950 (MI355X), one launch.
//
// Replaces the per-phase flash-attn calls of forward_mixed
// (nanovllm/layers/mixed_attention.py:36-57) and of the V0 branches of
// Attention.forward (nanovllm/layers/attention.py:68-78), and, with a bf16
// pool, the KV write that precedes them (attention.py:10-40): the launch then
// reads the step's new tokens from their rows and writes them to the pool as
// tail work (FOLD instantiations).
//
// Work list.  Every workgroup (4 wavefronts, two workgroups per CU) first
// derives, from the metadata alone, the number of work items of every row and
// their exclusive prefix (prefill rows first, then decode rows).  Item i
// belongs to list i % 8 and workgroup b serves list b % 8; the prefill items
// and the decode items of a list form two families, and workgroups start with
// one family or the other alternately so both phases begin at once.  Each list
// has a fetch counter on its own 128-byte line that is zero between launches:
// a launch makes a known number of fetches on it, and the workgroup that makes
// the last one resets it, so no memset is needed.  The grid is sized from
// capacities, never from device data, so the launch can be recorded in a HIP
// graph.
//
//  * Prefill item (row r, block of 16 or 32 query positions, kv head h): each
//    wavefront owns one of the G query heads that share kv head h, for the
//    same positions, so the K/V tiles staged in LDS serve all G heads.  The
//    block size is chosen per launch: 16 when the heaviest row's items would
//    otherwise outlast the balanced share of a workgroup, else 32 (E4M3FN
//    mixed launches also pick 16 per row for their longest rows).  Tiles
//    of 64 keys are double-buffered: the next tile's global loads are in
//    flight while the current one is consumed.  The contraction runs on bf16
//    MFMA (v_mfma_f32_16x16x32_bf16) in the transposed form S^T = K Q^T,
//    O^T += V^T P^T, which keeps each query column's softmax statistics
//    lane-local: the S^T accumulator is the B operand of the PV product
//    without data movement, and V^T comes from the natural [token][d] LDS tile
//    through ds_read_b64_tr_b16.
//  * Decode item (row b, chunk of 256 tokens, or 128 in launches with few
//    decode tokens, kv head h): four workgroup steps of 64 tokens, 16 per
//    wavefront; the G query heads sharing h are the MFMA columns.  K, V and Q
//    go from HBM straight into LDS (global_load_lds) and two steps stay in
//    flight per wavefront across item boundaries.  The 4 wavefronts merge in
//    LDS; a row with several chunks writes one (acc, m, l) record per chunk
//    and increments the (row, kv head) ticket.  After their items,
//    workgroups take tail tasks from their list: the folded KV write's
//    stores, and one merge task per (row, kv head), which waits until the
//    ticket counts every chunk and then merges the records (the split-K
//    merge of docs/project_manual.md:643-650).  That wait assumes every
//    workgroup of the launch is resident at once (the grid is the
//    instantiation's occupancy times the CUs); it is bounded (200 ms, or
//    SLO_ATTN_MERGE_WAIT_US), and a task that gives up writes NaN to its
//    outputs and counts the event, which slo_attention_workspace_check
//    reports.  Decode-only launches that fit a few rounds of workgroups run
//    decode_direct_kernel instead, where the workgroup whose chunk completes
//    a ticket merges: no workgroup waits for another there.
//
// LDS tiles are 64 rows of 256 bytes with the 16-byte chunks of each row
// XOR-swizzled (K: chunk ^ (row & 15); V: chunk ^ 2*(row & 7)), so the MFMA
// operand reads of 16 lanes fall on distinct banks.
//
// Split-K visibility across XCDs: partials are written and read with
// agent-scope stores/loads (global_store/load ... sc1), which bypass the
// per-XCD L2; each writer waits for its stores to be acknowledged and a
// workgroup barrier orders them before the ticket increment.  No L2 writeback
// or invalidate is needed.
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
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>
#include <mutex>
#include "common.h"
#include "capi_internal.h"
#include "tile_io.h"

namespace slo {

constexpr int NT = 256;                // threads per workgroup (4 wavefronts)
constexpr int TT = 64;                 // tokens per tile
constexpr int CHUNK = 256;             // decode split-K chunk (tokens): four workgroup steps
constexpr int CHUNK_MIN = 128;         // chunk of launches with few decode tokens (two live steps)
constexpr int TILE_BYTES = TT * ROWB;  // 16 KiB
constexpr int BQ_MIN = 16;             // query positions per prefill item: 16 or 32 (per launch)
constexpr int MAX_ROWS = 1024;         // decode + prefill rows per launch
constexpr int MAX_G = 16;              // query heads per kv head
constexpr int MAX_PAGES = 256;         // prefill block-table entries cached in LDS
constexpr int NLIST = 8;          // work lists (one per XCD)
constexpr int CTRL_STRIDE = 32;   // uint32 words between lists: one 128-byte line each
// Control area (4 KiB): three families of NLIST list lines (prefill items,
// decode items, tail tasks), one 128-byte line each, then a 1 KiB line whose
// first 528 bytes are the trash that decode wavefronts without a query head
// store to (so every wavefront issues the same number of stores per item)
// and whose last 128 bytes hold event counters (EV_*) that only the host's
// diagnostic reads and clears.  Every word of the list lines is zero between
// launches.
constexpr int TRASH_OFFSET = 3 * NLIST * CTRL_STRIDE * 4;
constexpr int TRASH_BYTES = 1024;
constexpr int EVENTS_OFFSET = TRASH_OFFSET + TRASH_BYTES - 128;
constexpr int CTRL_BYTES = TRASH_OFFSET + TRASH_BYTES;
enum : int {
  EV_MERGE_GAVE_UP = 0,   // split-K merge tasks that stopped waiting (their outputs are not written)
  EV_PF_SPLIT_MERGE = 1,  // split prefill item pairs merged by their second item
  EV_COUNT = 4,
};
constexpr int MAX_COUNTERS = 65536;
constexpr int PREC = HD + 4;      // floats per query head in a split-K record: acc[HD], m, l, 2 pad
constexpr size_t PARTIALS_OFFSET = CTRL_BYTES + sizeof(int) * (size_t)MAX_COUNTERS;
// Prefill-only launches may split their longest rows' items in two key
// ranges; each split item writes a record of its 4 wavefronts' (O, m, l) at
// the start of the partials area (unused by decode there), within this many
// bytes, which every workspace reserves beyond the decode partials.
constexpr size_t PF_SPLIT_BYTES = 48u << 20;
constexpr int PF_REC_FLOATS = 4 * (8 * 64 * 4 + 64 * 2);  // per item and 16 query positions
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
  int* ctrl;      // per list: [0] fetch counter (zero between launches)
  int* counters;  // split-K tickets, [num_decode * hkv]
  float* partials;
  // Query rows past every decode and prefill row of the arguments (whatever
  // the phases) start at q_off_prefill + cu_q_all[np_all]; they get zeros.
  const int32_t* cu_q_all;
  int32_t np_all;
  // KV write of the step's new tokens in this launch (bf16 pools; sslots is
  // null otherwise): new row t goes to slot sslots[t], and the launch reads
  // the new tokens from nk/nv (decode row b: row b; key j >= prefix of a
  // prefill row read through its table: its query row's index).
  const int32_t* sslots;
  const uint16_t* nk;
  const uint16_t* nv;
  int64_t nk_stride;
  int64_t nv_stride;
  int32_t nnew;
  int64_t num_slots;
  float scale_floor;  // E4M3FN pools with the KV write folded in: the store's scale_floor
  // How long a split-K merge task waits for its chunks before it gives up
  // (s_memrealtime ticks).
  int64_t merge_wait_ticks;
  // Bytes at the start of the partials area that split prefill items may use
  // for their records (prefill-only launches, which have no decode partials).
  int64_t pf_split_bytes;
};

// The two tile stages live in two separate __shared__ arrays of STAGE_BYTES
// (prefill: [K tile | V tile] of one buffer; decode: one DT-row V tile per
// wavefront).  Separate objects let the compiler see that a transposed LDS
// read of one stage cannot alias an LDS DMA still in flight to the other, so
// it does not drain the vector memory counter before that read.
constexpr int STAGE_BYTES = 2 * TILE_BYTES;

struct Smem {
  union {
    struct {
      float m[4][4];  // per wavefront, 4 query heads per pass
      float l[4][4];
      float sc[2][4][64];  // E4M3FN: K (0-31) and V (32-63) scales of a wavefront step, by stage
    } dec;                 // decode: cross-wavefront merge statistics
    struct {
      __attribute__((aligned(16))) float ks[2][TT];
      __attribute__((aligned(16))) float vs[2][TT];
      int pages[MAX_PAGES];  // block table of the current row
    } pf;                    // prefill
  } u;
  int off[MAX_ROWS + 1];
  int wsum[4];
  int wmax[4];
  int wumax[4];     // prefill-only set-up: key tiles of the longest block of a row that cannot split
  int dsum[4];
  uint32_t item;
  int row;
  int salt;
  int split_tiles;  // E4M3FN mixed launches: rows with a heavier 32-position block use 16
  int pf_first;     // workgroups that start with the prefill family
  int drot;         // decode items rotate kv heads across chunks (long decode launches)
  int pf_split_thr; // prefill-only launches: rows with a heavier block split their keys in two
  int pf_ticket;    // prefill split item: ticket value before this item's arrival
  int meta[2][20];  // decode: landed row length and block-table entries, by item parity
  int bcast[2];     // decode: row and local index of the item fetched by wavefront 0
  int kv_nt;        // decode K/V loads with the non-temporal cache policy
};


// The running max used as the exponent offset moves only when a tile's max
// exceeds it by more than 2^RESCALE_LOG2 (in units of the log2-scaled score),
// so every probability stays <= 2^RESCALE_LOG2 (exact in bf16's range, far
// from fp32 overflow in the row sum) and O is rescaled only on those rare
// tiles.  The result o / l is the same quantity as with an exact running max.
constexpr float RESCALE_LOG2 = 8.0f;

// Online softmax of one half tile (32 keys: score blocks sh[0], sh[1] hold key
// rows kh + 16*mm + 4g + i) for the wavefront's NQT query columns.  Scores stay
// unscaled until the exponent: max commutes with the positive factor
// c = softmax_scale*log2(e), so e = exp2(c*s - c*m) is one FMA and one
// v_exp_f32 per score; column reductions use v_permlane16/32_swap.  MASK
// selects the boundary-tile path (keys past the tile's valid rows or causally
// after the column).  SCALED (E4M3FN launches): scores take the keys' K scales
// and probabilities their V scales from ks/vs (1.0 for tiles of bf16 rows),
// without a per-score select.  Packs P^T into pb[nt] (the B operand of the half's PV
// product) and returns in alpha[nt] the factor the accumulators must take
// before that product; grow_any is set when any column's offset moved.
// Branch-free for bf16 sources, so the compiler can interleave it with MFMA
// work of the other half.
template <int NQT, bool MASK, bool SCALED>
__device__ __forceinline__ void softmax_half(f32x4 (&sh)[2][NQT], float (&m)[NQT], float (&l)[NQT], float (&alpha)[NQT],
                                             bool& grow_any, bf16x8 (&pb)[NQT], float c,
                                             const float* ks, const float* vs, int g, int ntok, int kh, int kv0,
                                             int lim0) {
  uint64_t grows = 0;
#pragma unroll
  for (int nt = 0; nt < NQT; ++nt) {
    if constexpr (SCALED) {
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) sh[mm][nt] *= *reinterpret_cast<const f32x4*>(ks + kh + 16 * mm + 4 * g);
    }
    if constexpr (MASK) {
      const int lim = lim0 + 16 * nt;
#pragma unroll
      for (int mm = 0; mm < 2; ++mm)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int tok = kh + 16 * mm + 4 * g + i;
          sh[mm][nt][i] = (tok < ntok && kv0 + tok <= lim) ? sh[mm][nt][i] : NEG_INF;
        }
    }
    float mx = NEG_INF;
#pragma unroll
    for (int mm = 0; mm < 2; ++mm)
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sh[mm][nt][i]);
    mx = col_max(mx);
    const bool grow = c * (mx - m[nt]) > RESCALE_LOG2;  // false when both are -inf
    const float mnew = grow ? mx : m[nt];
    const float cm = mnew == NEG_INF ? 0.0f : c * mnew;
    const float a = grow ? __builtin_amdgcn_exp2f(c * m[nt] - cm) : 1.0f;
    float rs = 0.0f;
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
      f32x4 vsc = f32x4{1, 1, 1, 1};
      if constexpr (SCALED) vsc = *reinterpret_cast<const f32x4*>(vs + kh + 16 * mm + 4 * g);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = __builtin_amdgcn_exp2f(fmaf(sh[mm][nt][i], c, -cm));
        rs += e;
        // (Boundary tiles: the V scales of keys past the valid ones are
        // whatever LDS holds there.)
        const float v = MASK && SCALED ? (kh + 16 * mm + 4 * g + i < ntok ? vsc[i] : 0.0f) : vsc[i];
        sh[mm][nt][i] = SCALED ? e * v : e;
      }
    }
    rs = col_sum(rs);
    l[nt] = l[nt] * a + rs;
    m[nt] = mnew;
    alpha[nt] = a;
    grows |= __builtin_amdgcn_ballot_w64(grow);
    u32x4 w;
    w.x = pack_bf16x2(sh[0][nt][0], sh[0][nt][1]);
    w.y = pack_bf16x2(sh[0][nt][2], sh[0][nt][3]);
    w.z = pack_bf16x2(sh[1][nt][0], sh[1][nt][1]);
    w.w = pack_bf16x2(sh[1][nt][2], sh[1][nt][3]);
    pb[nt] = as_bf16x8(w);
  }
  grow_any = grows != 0;
}

__device__ __forceinline__ int decode_len(const Params& p, int b) {
  const int L = p.dlens[b];
  return min(max(L, 0), p.dtab_width * p.block_size);
}

// Prefill row geometry: query range, usable keys and the bottom-right causal
// offset (keys before the first query position).
struct PfRow {
  int q_start, Lq, k_start, Lk, prefix;
};
__device__ __forceinline__ PfRow pf_row(const Params& p, int r) {
  PfRow g;
  g.q_start = p.cu_q[r];
  g.Lq = p.cu_q[r + 1] - g.q_start;
  g.k_start = p.cu_k[r];
  const int lk_full = p.cu_k[r + 1] - g.k_start;
  g.prefix = lk_full - g.Lq;
  int lk = lk_full;
  if (p.ptab != nullptr) lk = min(lk, p.ptab_width * p.block_size);
  else lk = min(lk, p.num_kv_rows - g.k_start);
  g.Lk = max(lk, 0);
  return g;
}

// Key tiles of the heaviest 32-position block of a prefill row, and an
// estimate of the row's total tile work (blocks x mean tiles x kv heads x
// head groups); `long_prefix`, when given, is set to whether the row's cached
// prefix is at least as long as its chunk (such rows may split, pf_splits).
__device__ __forceinline__ void pf_work(const Params& p, int r, int& work, int& tmax, bool* long_prefix = nullptr) {
  const PfRow g = pf_row(p, r);
  work = tmax = 0;
  if (long_prefix) *long_prefix = g.Lq > 0 && g.prefix >= g.Lq;
  if (g.Lq <= 0) return;
  const int nqb = (g.Lq + 31) / 32;
  tmax = (min(g.Lk, max(0, g.prefix + g.Lq)) + TT - 1) / TT;
  const int mean = (min(g.Lk, max(0, g.prefix + (g.Lq + 1) / 2)) + TT - 1) / TT;
  work = nqb * max(mean, 1) * p.hkv * p.HG;
}

__device__ __forceinline__ void store_partial(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Prefill-only launches split a row's items in two key ranges when its
// heaviest block spans more than `thr` key tiles and its cached prefix is at
// least as long as its chunk (measured: splitting cold rows made a launch of
// four 1.1k-token rows 5% slower, while rows after long prefixes gained).
__device__ __forceinline__ bool pf_splits(const Params& p, int r, int tiles, int thr) {
  if (tiles <= thr) return false;
  const PfRow g = pf_row(p, r);
  return g.prefix >= g.Lq;
}
// Prefill-only launches order their prefill items by the key count of the
// item's block, largest first, across rows: units (row, u) of hkv * HG items
// each (u = the row's block index counted from its heaviest block, times two
// with the halves of split rows) are ranked on the GPU.  Row geometry for the
// ranking: {prefix, Lq, usable keys, nqb | mult << 16}.
constexpr int PF_SORT_ROWS = 128;       // rows up to which the units are ranked
constexpr int PF_SORT_UNITS = 1024;     // units up to which they are ranked
constexpr int PF_SORT_COST = 1 << 14;   // units x rows up to which they are ranked
// Blocks of a row whose key count (min(Lk, max(0, prefix + min(bq (b + 1),
// Lq))), growing with b) exceeds K.
__device__ __forceinline__ int pf_blocks_above(const int4& g, int bq, int K) {
  const int nb = g.w & 0xffff;
  if (nb == 0) return 0;
  if (K < 0) return nb;
  if (g.z <= K || g.x + g.y <= K) return 0;
  const int x = K - g.x;
  if (x < 0) return nb;
  return max(0, nb - (x >> (bq == 32 ? 5 : 4)));  // x / bq (bq is 16 or 32)
}

__device__ __forceinline__ float load_partial(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- decode item
// A decode item (row b, kv head h, chunk c of CHUNK tokens) is NSTEP = 4
// workgroup steps of DSTEP tokens; in step s wavefront w takes the DT tokens
// starting at c*CHUNK + s*DSTEP + w*DT (E4M3FN pools: twice as many tokens per
// wavefront, step and item, d_dt and d_chunk).  A wavefront step lies in one
// KV block (block_size is a multiple of 64).  Step s uses LDS stage s & 1, private to
// each wavefront, and the item's Q goes to one half of a double-buffered LDS
// array, so K, V and Q all go HBM -> LDS through global_load_lds_dwordx4 and
// no streamed data is held in registers across iterations.  Two steps are in
// flight per wavefront at all times, across item boundaries.
//
// Every vector memory operation of the loop (LDS DMA, atomics, split-K and
// output stores) is issued through inline assembly at a fixed point, in the
// same number on every pass: a wavefront step past the row's length issues
// its operations as single-lane 4-byte loads, after the last item
// the next-item loads repeat the current item's, a ticket with nothing due
// adds 0, a fetch after the list's end adds 0, and a wavefront without a query
// head stores to a trash line.  Vector memory operations complete in issue
// order, so every wait is an exact `s_waitcnt vmcnt(N)` whose N counts the
// operations issued after the awaited ones, and no wait covers an operation
// issued for a later step.  (The compiler's own bookkeeping cannot follow
// loads that land in LDS and would drain the pipeline.)  Wavefront 0 alone
// fetches work, finds the fetched item's row, loads its length and
// block-table entries into LDS and broadcasts the row; the fetch and ticket
// results are read after a wait that covers them, through an empty asm that
// ties the value to that point.
//
// Split-K: an item of a row with several chunks stores its record, and once
// the stores of every wavefront are acknowledged (the wait and barrier of the
// next item's step 1) wavefront 0 adds 1 to the (row, kv head) ticket; the
// merge is a tail task (tail_tasks).
constexpr int DT = 16;                 // tokens per wavefront step
constexpr int DSTEP = 4 * DT;          // tokens per workgroup step
constexpr int NSTEP = CHUNK / DSTEP;   // workgroup steps per item
constexpr int WSTAGE = 2 * DT * ROWB;  // per wavefront and stage: K rows, then V rows (bf16)
constexpr int QBUF = MAX_G * HD * 2;   // bytes of one half of the Q buffer
static_assert(NSTEP == 4, "the decode loop is written for four workgroup steps per item");
static_assert(4 * WSTAGE <= STAGE_BYTES, "decode stage must fit the tile stage");

// E4M3FN pools take 32 tokens per wavefront step (two 16-token halves, the
// same bytes as 16 bf16 tokens), so a wavefront keeps as many bytes in flight
// as with bf16 and an item of four steps spans 512 tokens.
template <bool FP8>
__host__ __device__ __forceinline__ constexpr int d_dt() { return FP8 ? 2 * DT : DT; }  // tokens per wavefront step
template <bool FP8>
__host__ __device__ __forceinline__ constexpr int d_step() { return 4 * d_dt<FP8>(); }  // tokens per workgroup step
template <bool FP8>
__host__ __device__ __forceinline__ constexpr int d_chunk() { return NSTEP * d_step<FP8>(); }  // tokens per item
template <bool FP8>
__host__ __device__ __forceinline__ constexpr int d_chunk_min() { return d_chunk<FP8>() / 2; }  // two live steps
// Vector memory operations per wavefront step: bf16 4 K + 4 V; E4M3FN 4 K
// codes + 4 V codes + 1 of scales, and with the KV write folded in 1 of the
// row's new K and V.
template <bool FP8, bool FOLD>
__device__ __forceinline__ constexpr int d_group() { return FP8 ? (FOLD ? 10 : 9) : 8; }

struct DMeta {
  int b, h, c, dindex;  // wave-uniform
  int tok0, span;       // first token of the item, tokens per item (the launch's chunk)
  int len;              // dlens[b] as read (clamped where used)
  int page[NSTEP];      // KV block of each workgroup step
};

__device__ __forceinline__ int decode_L(const Params& p, const DMeta& m) {
  return min(max(m.len, 0), p.dtab_width * p.block_size);
}
__device__ __forceinline__ int decode_nch(const Params& p, const DMeta& m) {
  return max(1, (decode_L(p, m) + m.span - 1) / m.span);
}

// Item geometry from its row and index within the row.
// With rot, chunk c of a row takes kv head (j + c) % hkv for local index
// c * hkv + j, so each work list cycles through the heads instead of keeping
// one (its record keeps the slot of its (chunk, head)).
__device__ __forceinline__ DMeta decode_geom(const Params& p, int r, int local, int item, int decode_base,
                                             int dchunk, bool rot) {
  DMeta m;
  m.b = r - p.np;
  m.c = local / p.hkv;
  m.h = rot ? (local % p.hkv + m.c) % p.hkv : local % p.hkv;
  m.dindex = item - decode_base - local + m.c * p.hkv + m.h;
  m.span = dchunk;
  m.tok0 = m.c * dchunk;
  m.len = 0;
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) m.page[s] = -1;
  return m;
}
// Wavefront 0: one LDS DMA of the item's row length (lane 0) and the
// block-table entries of its steps (bf16: lanes 1..NSTEP, one per workgroup
// step; E4M3FN: lanes 1..4*NSTEP, one per step and wavefront, since a
// 128-token workgroup step may span two blocks of 64) into sm.meta[slot].  It
// is counted by vmcnt like the KV loads.  (Scalar loads would share lgkmcnt
// with LDS, so the next LDS wait would stall on their latency; a load into a
// VGPR could be copied by the compiler before it lands.)
template <bool FP8>
__device__ __forceinline__ void decode_meta_dma(const Params& p, Smem& sm, const DMeta& m, int slot, int lane) {
  constexpr int NE = FP8 ? 4 * NSTEP : NSTEP;  // table entries
  const int e = lane - 1;
  const int tok = FP8 ? m.tok0 + (e >> 2) * d_step<FP8>() + (e & 3) * d_dt<FP8>() : m.tok0 + e * DSTEP;
  const int32_t* src = (e >= 0 && e < NE)
                           ? p.dtab + (int64_t)m.b * p.dtab_stride + min(tok / p.block_size, p.dtab_width - 1)
                           : p.dlens + m.b;
  if (lane <= NE) dma4(src, lds_addr(sm.meta[slot]));
}
// After a wait that covers the DMA and a barrier.  page[s] is the block of
// this wavefront's tokens of step s.
template <bool FP8>
__device__ __forceinline__ void decode_meta_read(DMeta& m, const Smem& sm, int slot, int wave) {
  m.len = __builtin_amdgcn_readfirstlane(sm.meta[slot][0]);
#pragma unroll
  for (int s = 0; s < NSTEP; ++s)
    m.page[s] = __builtin_amdgcn_readfirstlane(sm.meta[slot][1 + (FP8 ? 4 * s + wave : s)]);
}

// Decode items of a list.  With group = hkv (E4M3FN pools) the kv heads of
// one (row, chunk) are consecutive items of the family and go to one list
// together, so the workgroups reading one chunk's heads share an XCD and its
// L2: each head's scales are 4 of every hkv*4 bytes of the scale rows, whose
// lines the heads then fetch from HBM once instead of once each (measured
// 95.7 -> 87.0 us on 64 rows of 512-4096 tokens).  With group = 1 (bf16, no
// gain there) item x of the family is on list x % nlist.  Group g = x / group
// is on list g % nlist, at relative index (g / nlist) * group + x % group.
__device__ __forceinline__ int dec_index(int list, int nlist, int group, int rel) {
  return ((rel / group) * nlist + list) * group + rel % group;
}
__device__ __forceinline__ int dec_count(int list, int nlist, int group, int size) {
  const int groups = size / group;
  return list < groups ? ((groups - list + nlist - 1) / nlist) * group : 0;
}

// Row of item `item` among rows [lo, nrows), searched by one wavefront.
__device__ __forceinline__ int find_row(const Smem& sm, int item, int lo, int nrows, int lane) {
  for (int base = lo; base < nrows; base += 64) {
    const int r = base + lane;
    const bool hit = r < nrows && sm.off[r] <= item && item < sm.off[r + 1];
    const uint64_t mask = __builtin_amdgcn_ballot_w64(hit);
    if (mask) return base + (int)__builtin_ctzll(mask);
  }
  return -1;
}

// Valid tokens of wavefront `wave` in step s of the item (0 for padding
// blocks and for steps past the item's span).
template <bool FP8>
__device__ __forceinline__ int decode_ntok(const Params& p, const DMeta& m, int s, int wave) {
  const int page = m.page[s];
  if (page < 0 || page >= p.num_blocks || s * d_step<FP8>() >= m.span) return 0;
  return min(max(decode_L(p, m) - (m.tok0 + s * d_step<FP8>() + wave * d_dt<FP8>()), 0), d_dt<FP8>());
}

// The item's G query heads (G*HD bf16, contiguous in the row) to qbuf; each
// wavefront copies one quarter.
__device__ __forceinline__ void decode_issue_q(const Params& p, uint8_t* qbuf, const DMeta& m, int wave, int lane) {
  const int qb = 64 * p.G;  // bytes per wavefront
  const uint8_t* src = reinterpret_cast<const uint8_t*>(p.q + (int64_t)m.b * p.q_stride + (int64_t)m.h * p.G * HD);
  const uint32_t dst = lds_addr(qbuf + wave * qb);
  if (lane < 4 * p.G) dma16(src + wave * qb + 16 * lane, dst);
}

// K and V of one wavefront step to the wavefront's stage region `stg`.
// bf16: K row r at r*ROWB with 16-byte chunk c in slot c ^ (r & 15), V rows
// from 4*ROWB*4 on with chunk c in slot c ^ 2*(r & 7).  E4M3FN (32 tokens):
// see below; the scales go to `scl`.  NT: the K/V (code) bytes are loaded
// with the non-temporal cache policy, which streams them faster (each line is
// read once, whole).
template <bool FP8, bool FOLD, bool NT = true>
__device__ __forceinline__ void decode_issue(const Params& p, uint8_t* stg, float* scl, uint8_t* nrw, const DMeta& m,
                                             int s, int wave, int lane) {
  const int n = lane & 15, g = lane >> 4;
  const int ntok = decode_ntok<FP8>(p, m, s, wave);
  const int t0 = m.tok0 + s * d_step<FP8>() + wave * d_dt<FP8>();
  if (ntok == 0) {
    // A step without valid tokens issues the same number of operations, each
    // a 4-byte load on one lane: counted like the others, nearly free.
    const uint32_t dst = lds_addr(stg);
    if (lane == 0) {
#pragma unroll
      for (int i = 0; i < d_group<FP8, FOLD>(); ++i) dma4(p.dlens, dst + 4 * i);
    }
    return;
  }
  const int64_t slot0 = (int64_t)m.page[s] * p.block_size + t0 % p.block_size;
  const int row = p.hkv * HD;  // elements (bf16) or bytes (E4M3FN) between tokens
  const int64_t base = slot0 * row + (int64_t)m.h * HD;
  if constexpr (!FP8) {
    const uint16_t* kc = static_cast<const uint16_t*>(p.k_cache) + base;
    const uint16_t* vc = static_cast<const uint16_t*>(p.v_cache) + base;
    const uint32_t dst = lds_addr(stg);
    // With the KV write in this launch, the row's newest token (its last) is
    // read from the new rows: its slot is written by this same launch.
    const int tnew = FOLD ? decode_L(p, m) - 1 - t0 : -1;  // its row in this step, if any
    const uint16_t* kn = FOLD ? p.nk + (int64_t)m.b * p.nk_stride + m.h * HD : kc;
    const uint16_t* vn = FOLD ? p.nv + (int64_t)m.b * p.nv_stride + m.h * HD : vc;
    auto load = [&](auto policy_nt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * i + g;
        const uint16_t* src = (r == tnew ? kn : kc + r * row) + 8 * (n ^ (r & 15));
        if constexpr (decltype(policy_nt)::value) dma16_nt(src, dst + i * 1024);
        else dma16(src, dst + i * 1024);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * i + g;
        const uint16_t* src = (r == tnew ? vn : vc + r * row) + 8 * (n ^ ((r & 7) << 1));
        if constexpr (decltype(policy_nt)::value) dma16_nt(src, dst + DT * ROWB + i * 1024);
        else dma16(src, dst + DT * ROWB + i * 1024);
      }
    };
    load(std::integral_constant<bool, NT>());
  } else {
    // 32 tokens: rows 16h..16h+15 go to half h at 4096h (K codes, 128-byte
    // rows with 16-byte chunk c in slot c ^ (r & 7), then V codes at +2048);
    // the K and V scales to scl[0..31] and scl[32..63].
    const uint8_t* kc = static_cast<const uint8_t*>(p.k_cache) + base;
    const uint8_t* vc = static_cast<const uint8_t*>(p.v_cache) + base;
    const uint32_t dst = lds_addr(stg);
    auto load = [&](auto policy_nt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 8 * i + (lane >> 3);
        const uint8_t* src = kc + r * row + 16 * ((lane & 7) ^ (r & 7));
        if constexpr (decltype(policy_nt)::value) dma16_nt(src, dst + (i >> 1) * 4096 + (i & 1) * 1024);
        else dma16(src, dst + (i >> 1) * 4096 + (i & 1) * 1024);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 8 * i + (lane >> 3);
        const uint8_t* src = vc + r * row + 16 * ((lane & 7) ^ (r & 7));
        if constexpr (decltype(policy_nt)::value) dma16_nt(src, dst + (i >> 1) * 4096 + 2048 + (i & 1) * 1024);
        else dma16(src, dst + (i >> 1) * 4096 + 2048 + (i & 1) * 1024);
      }
    };
    load(std::integral_constant<bool, NT>());
    const float* sc = (lane & 32) ? p.v_scale : p.k_scale;
    dma4(sc + (slot0 + (lane & 31)) * p.hkv + m.h, lds_addr(scl));
    if constexpr (FOLD) {
      // The row's new K (lanes 0-15) and V (lanes 16-31) of head h, bf16, to
      // nrw: the newest token's slot is written only at the launch's end, so
      // its codes are made from them (decode_wstep).  Every step loads them.
      const uint16_t* src = ((lane & 16) ? p.nv + (int64_t)m.b * p.nv_stride : p.nk + (int64_t)m.b * p.nk_stride) +
                            m.h * HD + 8 * (lane & 15);
      if (lane < 32) dma16(src, lds_addr(nrw));
    }
  }
}

// QK, online softmax and PV of one landed bf16 step (16 tokens) into this
// wavefront's running (o, m, l); lane (n, g) holds O^T[d = 16dt + 4g + i][head
// n] and the statistics of head n.  Scores are in the log2 domain.
__device__ __forceinline__ void decode_step_bf16(const Params& p, const uint8_t* stg, int ntok, const u32x4 (&qv)[4],
                                                 f32x4 (&o)[8], float& m, float& l, int lane) {
  const int n = lane & 15, g = lane >> 4;
  const uint8_t* vt = stg + DT * ROWB;

  // V^T operand: source lane n of group g reads row 4g + n/4, d = 16dt + 4(n%4).
  // Every LDS operand read of the step (4 K, 8 V^T fragments) is issued
  // before the first MFMA, so the step pays one LDS round trip.
  const int r0 = 4 * g + (n >> 2);
  s16x4 va[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) va[dt] = lds_tr16(vt + v_off(r0, 2 * dt + ((n & 3) >> 1)) + ((n & 1) << 3));
  // S^T = K Q^T for the 16 tokens: k-step kk covers d = 32kk + 8g + {0..7}.
  u32x4 a[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) a[kk] = ld16(stg + k_off(n, 4 * kk + g));
  f32x4 s = f32x4{0, 0, 0, 0};
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) s = mfma16(as_bf16x8(a[kk]), as_bf16x8(qv[kk]), s);

  if (ntok < DT) {
    // V rows past the valid tokens (whatever the pool holds there) become
    // zeros in the operand: lane (n, g) holds tokens 4g + {0..3}.
    const uint32_t m01 = (4 * g + 0 < ntok ? 0xffffu : 0u) | (4 * g + 1 < ntok ? 0xffff0000u : 0u);
    const uint32_t m23 = (4 * g + 2 < ntok ? 0xffffu : 0u) | (4 * g + 3 < ntok ? 0xffff0000u : 0u);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const u32x2 w = __builtin_bit_cast(u32x2, va[dt]);
      va[dt] = __builtin_bit_cast(s16x4, u32x2{w.x & m01, w.y & m23});
    }
  }

  float x[4];
  float mx = NEG_INF;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[i] = 4 * g + i < ntok ? s[i] * p.scale_log2 : NEG_INF;
    mx = fmaxf(mx, x[i]);
  }
  mx = col_max(mx);
  // Lazy offset (as in the prefill softmax): it moves only by more than
  // 2^RESCALE_LOG2, so e <= 2^RESCALE_LOG2 and O is rarely rescaled.
  const bool grow = mx - m > RESCALE_LOG2;  // false when both are -inf
  const float mnew = grow ? mx : m;
  const float mu = mnew == NEG_INF ? 0.0f : mnew;
  const float alpha = grow ? __builtin_amdgcn_exp2f(m - mu) : 1.0f;
  float e[4], rs = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    e[i] = __builtin_amdgcn_exp2f(x[i] - mu);
    rs += e[i];
  }
  rs = col_sum(rs);
  l = l * alpha + rs;
  m = mnew;
  if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt] *= alpha;
  }
  // P^T as the B operand of the 16x16x16 product: k slot (g, j) is token 4g + j.
  // P goes in as two bf16 terms, hi = bf16(e) and lo = bf16(e - hi) (the
  // difference is exact in fp32), so the product carries P to about 2^-17
  // relative instead of bf16's 2^-9.  The stream is HBM-bound; the second
  // product costs MFMA cycles that are idle anyway.
  const uint32_t h01 = pack_bf16x2(e[0], e[1]), h23 = pack_bf16x2(e[2], e[3]);
  const s16x4 pb = __builtin_bit_cast(s16x4, u32x2{h01, h23});
  const s16x4 pl = __builtin_bit_cast(s16x4, u32x2{
      pack_bf16x2(e[0] - __uint_as_float(h01 << 16), e[1] - __uint_as_float(h01 & 0xffff0000u)),
      pack_bf16x2(e[2] - __uint_as_float(h23 << 16), e[3] - __uint_as_float(h23 & 0xffff0000u))});
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va[dt], pb, o[dt], 0, 0, 0);
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va[dt], pl, o[dt], 0, 0, 0);
}

// 8-byte transposed LDS read: lane (2j + c) of each 16-lane group passes the
// address of bytes 8c..8c+7 of row j of an 8 x 16-byte block; lane n gets
// byte n of rows 0..7 (byte j = row j).
__device__ __forceinline__ u32x2 lds_tr8(const uint8_t* p) {
  typedef int v2i __attribute__((vector_size(8)));
  const v2i r = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i*)(const_cast<uint8_t*>(p)));
  return u32x2{(uint32_t)r[0], (uint32_t)r[1]};
}

// E4M3FN step of 32 tokens (the wavefront's codes: token t at half t / 16,
// row t % 16 of stg, K codes at 4096 * half, V codes 2048 further; scales
// ksp/vsp[t]).  The scores are made in two 16x16 products whose row r is
// token 8 (r / 4) + 4h + r % 4 (half h), so lane (n, g) holds the scores of
// tokens 8g..8g+7 of head n: one softmax update for the 32 tokens, and P^T
// is the B operand of 16x16x32 products as it stands.  The V^T operand (row
// d, tokens 8g..8g+7) comes straight from the codes by a transposed byte
// read, masked to the valid tokens and converted in registers.
__device__ __forceinline__ void decode_step_e4m3(const Params& p, const uint8_t* stg, const float* ksp,
                                                 const float* vsp, int ntok, const u32x4 (&qv)[4], f32x4 (&o)[8],
                                                 float& m, float& l, int lane) {
  const int n = lane & 15, g = lane >> 4;
  f32x4 s[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int t = 8 * (n >> 2) + 4 * h + (n & 3), rr = t & 15;
    const uint8_t* kr = stg + (t >> 4) * 4096 + rr * 128;
    u32x4 a[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int c = 2 * kk + (g >> 1);
      a[kk] = fp8x8_to_bf16x8(ld8(kr + 16 * (c ^ (rr & 7)) + 8 * (g & 1)));
    }
    s[h] = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) s[h] = mfma16(as_bf16x8(a[kk]), as_bf16x8(qv[kk]), s[h]);
  }
  // V^T fragments: lane (n, g) addresses row n / 2 (token 8g + n / 2), bytes
  // 8 (n % 2).. of d-chunk dt.
  const int tv = 8 * g + (n >> 1), rv = tv & 15;
  const uint8_t* vr = stg + (tv >> 4) * 4096 + 2048 + rv * 128 + 8 * (n & 1);
  u32x2 vc[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) vc[dt] = lds_tr8(vr + 16 * (dt ^ (rv & 7)));
  const f32x4 k0 = __builtin_bit_cast(f32x4, ld16(ksp + 8 * g)), k1 = __builtin_bit_cast(f32x4, ld16(ksp + 8 * g + 4));
  const f32x4 v0 = __builtin_bit_cast(f32x4, ld16(vsp + 8 * g)), v1 = __builtin_bit_cast(f32x4, ld16(vsp + 8 * g + 4));
  const int nv = min(max(ntok - 8 * g, 0), 8);  // valid tokens of this lane's 8
  float x[8];
  float mx = NEG_INF;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[i] = i < nv ? s[0][i] * p.scale_log2 * k0[i] : NEG_INF;
    x[4 + i] = 4 + i < nv ? s[1][i] * p.scale_log2 * k1[i] : NEG_INF;
    mx = fmaxf(mx, fmaxf(x[i], x[4 + i]));
  }
  mx = col_max(mx);
  const bool grow = mx - m > RESCALE_LOG2;  // false when both are -inf
  const float mnew = grow ? mx : m;
  const float mu = mnew == NEG_INF ? 0.0f : mnew;
  const float alpha = grow ? __builtin_amdgcn_exp2f(m - mu) : 1.0f;
  float e[8], rs = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    e[i] = __builtin_amdgcn_exp2f(x[i] - mu);
    rs += e[i];
    // Scales of tokens past the valid ones are whatever LDS holds there.
    e[i] = i < nv ? e[i] * (i < 4 ? v0[i] : v1[i - 4]) : 0.0f;
  }
  rs = col_sum(rs);
  l = l * alpha + rs;
  m = mnew;
  if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt] *= alpha;
  }
  u32x4 hi, lo;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t h2 = pack_bf16x2(e[2 * j], e[2 * j + 1]);
    hi[j] = h2;
    lo[j] = pack_bf16x2(e[2 * j] - __uint_as_float(h2 << 16), e[2 * j + 1] - __uint_as_float(h2 & 0xffff0000u));
  }
  // Codes of tokens past the valid ones may be NaN patterns: zeroed.
  const uint64_t keep = nv >= 8 ? ~0ull : (1ull << (8 * nv)) - 1;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    const uint32_t w0 = vc[dt].x & (uint32_t)keep, w1 = vc[dt].y & (uint32_t)(keep >> 32);
    const u32x4 va = fp8x8_to_bf16x8(u32x2{w0, w1});
    o[dt] = mfma16(as_bf16x8(va), as_bf16x8(hi), o[dt]);
    o[dt] = mfma16(as_bf16x8(va), as_bf16x8(lo), o[dt]);
  }
}

// One wavefront step: 16 bf16 tokens, or 32 E4M3FN tokens.
template <bool FP8, bool FOLD>
__device__ __forceinline__ void decode_wstep(const Params& p, uint8_t* stg, float* scl, const uint8_t* nrw, int ntok,
                                             int tnew, const u32x4 (&qv)[4], f32x4 (&o)[8], float& m, float& l,
                                             int lane) {
  if constexpr (FP8 && FOLD) {
    // With the KV write folded in, the row's newest token (row tnew of this
    // step, when it holds it) gets the codes and scales the store writes, made
    // here from its new K and V as slo_store_kvcache makes them (lanes 32-63
    // repeat lanes 0-31).
    if (tnew >= 0 && tnew < ntok) {
      const u32x4 x = ld16(nrw + 16 * (lane & 31));
      float f[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f[2 * j] = bf16_bits_to_f32(x[j] & 0xffffu);
        f[2 * j + 1] = bf16_bits_to_f32(x[j] >> 16);
      }
      float sc;
      const u32x2 codes = e4m3_encode8<16>(f, p.scale_floor, sc);
      if (lane < 32) {
        const int isv = lane >> 4, c8 = lane & 15, rl = tnew & 15;
        uint8_t* row = stg + (tnew >> 4) * 4096 + isv * 2048 + rl * 128;
        *reinterpret_cast<u32x2*>(row + 16 * ((c8 >> 1) ^ (rl & 7)) + 8 * (c8 & 1)) = codes;
        if (c8 == 0) scl[isv * 32 + tnew] = sc;
      }
    }
  }
  if constexpr (FP8) {
    decode_step_e4m3(p, stg, scl, scl + 32, ntok, qv, o, m, l, lane);
  } else {
    decode_step_bf16(p, stg, ntok, qv, o, m, l, lane);
  }
}

// Cross-wavefront merge.  Per pass of 4 query heads, every wavefront writes
// its accumulators into its own stage-1 region (idle between its last step
// and the next item's step-1 loads) and its (m, l) into the merge area; after
// a barrier, wavefront w combines query head 4*pass + w over the four
// wavefronts (lane j < 32 owns d = 4j..4j+3) and writes the output (single
// chunk) or the chunk's split-K record [acc | m, l] (lane 32 holds m, l).
// Every wavefront issues exactly one store instruction per pass (to the trash
// line when it has no head), so the decode loop's waits can count them.
// Entered after a barrier that follows every wavefront's last step; ends with
// a barrier, after which the stage-1 regions may take new loads.
__device__ __forceinline__ void decode_merge(const Params& p, Smem& sm, uint8_t* st1, const DMeta& md, int tid,
                                             const f32x4 (&o)[8], float mx, float ls) {
  const int lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int G = p.G;
  const int nch = decode_nch(p, md);
  float* part = p.partials + (size_t)md.dindex * G * PREC;
  float* own = reinterpret_cast<float*>(st1 + wave * WSTAGE);  // [4 heads][HD]
  for (int hg = 0; hg < G; hg += 4) {
    if (hg > 0) lds_sync();
    if (n >= hg && n < min(G, hg + 4)) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<f32x4*>(own + (n - hg) * HD + 16 * dt + 4 * g) = o[dt];
      if (g == 0) {
        sm.u.dec.m[wave][n - hg] = mx;
        sm.u.dec.l[wave][n - hg] = ls;
      }
    }
    lds_sync();
    const int hn = hg + wave;
    const int j = lane & 31;
    if (hn >= G) {
      if (lane < 33) store16(reinterpret_cast<uint8_t*>(p.ctrl) + TRASH_OFFSET + 16 * lane, u32x4{0, 0, 0, 0});
      continue;
    }
    float M = NEG_INF;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, sm.u.dec.m[w][wave]);
    float Ls = 0.0f;
    f32x4 acc = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float mw = sm.u.dec.m[w][wave];
      const float f = mw == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
      Ls += f * sm.u.dec.l[w][wave];
      acc += f * *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(st1 + w * WSTAGE) + wave * HD + 4 * j);
    }
    if (nch == 1) {
      const float inv = Ls > 0.0f ? 1.0f / Ls : 0.0f;
      if (lane < 32)
        store8(p.out + (int64_t)md.b * p.out_stride + (int64_t)(md.h * G + hn) * HD + 4 * j,
               u32x2{pack_bf16x2(acc[0] * inv, acc[1] * inv), pack_bf16x2(acc[2] * inv, acc[3] * inv)});
    } else if (lane < 33) {
      const f32x4 v = lane < 32 ? acc : f32x4{M, Ls, 0.0f, 0.0f};
      store16_agent(part + hn * PREC + 4 * lane, __builtin_bit_cast(u32x4, v));
    }
  }
  lds_sync();
}

// Final split-K merge of (row b, kv head h): a thread owns one query head and
// two adjacent d; the chunks' (m, l) and accumulator pairs are read 16 chunks
// at a time (agent-scope 8-byte loads), merged online, and the ticket reset.
// Run once the ticket counts every chunk: every record is stored and
// acknowledged before its increment, and the loads bypass the per-XCD L2.
__device__ __forceinline__ float2 load_partial2(const float* p) {
  const uint64_t v = __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<float*>(p)), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  return __builtin_bit_cast(float2, v);
}

__device__ __forceinline__ void decode_final(const Params& p, int b, int h, int dfirst, int nch, int tid) {
  const int G = p.G;
  const size_t pstride = (size_t)p.hkv * G * PREC;  // floats between chunks of one (row, head)
  const float* p0 = p.partials + (size_t)dfirst * G * PREC;
  for (int u = tid; u < G * (HD / 2); u += NT) {
    const int hn = u / (HD / 2), d = 2 * (u % (HD / 2));
    float M = NEG_INF, Ls = 0.0f, O0 = 0.0f, O1 = 0.0f;
    for (int c0 = 0; c0 < nch; c0 += 16) {
      float2 ml[16], ov[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const bool ok = c0 + k < nch;
        const float* pc = p0 + (size_t)(ok ? c0 + k : c0) * pstride;
        ml[k] = ok ? load_partial2(pc + hn * PREC + HD) : make_float2(NEG_INF, 0.0f);
        ov[k] = ok ? load_partial2(pc + hn * PREC + d) : make_float2(0.0f, 0.0f);
      }
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const float mn = fmaxf(M, ml[k].x);
        if (mn == NEG_INF) continue;
        const float a = __builtin_amdgcn_exp2f(M - mn), bw = __builtin_amdgcn_exp2f(ml[k].x - mn);
        Ls = Ls * a + ml[k].y * bw;
        O0 = O0 * a + ov[k].x * bw;
        O1 = O1 * a + ov[k].y * bw;
        M = mn;
      }
    }
    const float inv = Ls > 0.0f ? 1.0f / Ls : 0.0f;
    *reinterpret_cast<uint32_t*>(p.out + (int64_t)b * p.out_stride + (int64_t)(h * G + hn) * HD + d) =
        pack_bf16x2(O0 * inv, O1 * inv);
  }
  // The launch's nch increments are matched by one decrement of nch: the
  // ticket is zero for the next launch whatever the order.
  if (tid == 0) __hip_atomic_fetch_add(&p.counters[b * p.hkv + h], -nch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// KV write of new-row pieces [first, end) (16-byte pieces, a new row's K
// pieces then its V pieces): each copied to the row's slot (slots < 0 or past
// the pool are skipped), all loads of the call first, then the stores; the
// E4M3FN pool gets the quantising store of slo_store_kvcache.  Thread tid
// takes pieces first + tid + j * NT (j < 4); with first a multiple of 16, the
// 16 lanes of one (token, kv head) vector are whole groups.
template <bool FP8>
__device__ __forceinline__ void store_new_rows(const Params& p, int64_t first, int64_t end, int tid) {
  const int row = p.hkv * HD;  // elements of one K (or V) row
  const int per_tok = 2 * (row / 8);
  for (int64_t i0 = first; i0 < end; i0 += 4 * NT) {
    u32x4 x[4];
    int64_t dst[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t i = i0 + tid + j * NT;
      const int64_t t = i / per_tok;
      const int pc = (int)(i % per_tok);
      const bool isv = pc >= row / 8;
      const int e = 8 * (isv ? pc - row / 8 : pc);
      dst[j] = -1;
      x[j] = u32x4{0, 0, 0, 0};
      if (i < end) {
        const int64_t slot = p.sslots[t];
        x[j] = ld16((isv ? p.nv + t * p.nv_stride : p.nk + t * p.nk_stride) + e);
        if (slot >= 0 && slot < p.num_slots) dst[j] = 2 * (slot * row + e) + (isv ? 1 : 0);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (FP8) {
        // The 16 lanes of one (token, kv head) vector (whole groups: pieces
        // and the token are the same across them) share its amax.
        float f[8];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          f[2 * k] = bf16_bits_to_f32(x[j][k] & 0xffffu);
          f[2 * k + 1] = bf16_bits_to_f32(x[j][k] >> 16);
        }
        float sc;
        const u32x2 codes = e4m3_encode8<HD / 8>(f, p.scale_floor, sc);
        if (dst[j] < 0) continue;
        const int64_t e = dst[j] >> 1;  // element (= byte) offset slot * row + d
        uint8_t* base = static_cast<uint8_t*>(const_cast<void*>((dst[j] & 1) ? p.v_cache : p.k_cache));
        *reinterpret_cast<u32x2*>(base + e) = codes;
        if ((e % HD) == 0) const_cast<float*>((dst[j] & 1) ? p.v_scale : p.k_scale)[e / HD] = sc;
      } else {
        if (dst[j] < 0) continue;
        uint16_t* base = static_cast<uint16_t*>(const_cast<void*>((dst[j] & 1) ? p.v_cache : p.k_cache));
        *reinterpret_cast<u32x4*>(base + (dst[j] >> 1)) = x[j];
      }
    }
  }
}

// Tail tasks, taken by each workgroup once its items are done: first the KV
// write of the launch's new tokens (when the launch carries it), then the
// split-K merges.  Store task i of list l writes new rows [4g, 4g + 4) for
// g = l + i * nlist: each K and V row is copied to its slot (slots < 0 or
// past the pool are skipped).  Nothing in the launch reads those slots before
// writing them (the new tokens are read from the new rows; a prefill item
// whose prefix ends inside a key tile first writes that tile's new tokens
// itself, the same bytes), so the writes need no ordering and the workgroups
// that finish their items first do them.  Merge tasks, one per (decode row,
// kv head) in row-major order, are spread over the work lists (task t on
// list t % nlist).  A merge task waits until all chunk tickets of its (row,
// head) have arrived (each chunk increments the ticket only after its record
// is stored, and chunks are run by workgroups that are resident: the grid is
// what the GPU holds of this instantiation at once), merges, and takes nch
// off the ticket.  The wait is bounded by merge_wait_ticks (200 ms); a task
// that gives up writes nothing, takes nch off the ticket all the same (the
// late increments bring it back to zero, so the next launch is unaffected)
// and counts the event, which slo_attention_workspace_check reports as an
// error.  Like the work lists, the task counter starts at zero: a launch
// makes exactly tasks + workgroups fetches on it, and the workgroup making
// the last one resets it.
constexpr int STORE_ROWS = 4;  // new rows per store task
template <bool FP8, bool STORE>
__device__ void tail_tasks(const Params& p, Smem& sm, int list, int nlist, int decode_base, int dchunk, int tid) {
  uint32_t* mctr = reinterpret_cast<uint32_t*>(p.ctrl) + (2 * NLIST + list) * CTRL_STRIDE;
  const int ngroups = STORE ? (p.nnew + STORE_ROWS - 1) / STORE_ROWS : 0;
  const uint32_t nstore = list < ngroups ? (uint32_t)((ngroups - list + nlist - 1) / nlist) : 0u;
  const int ntask = p.nd * p.hkv;
  const uint32_t count = nstore + (list < ntask ? (uint32_t)((ntask - list + nlist - 1) / nlist) : 0u);
  const uint32_t wgs = (uint32_t)((gridDim.x - list + nlist - 1) / nlist);
  if (count == 0) return;  // a list without tasks is not touched: its counter stays zero
  const int per_tok = 2 * (p.hkv * HD / 8);  // 16-byte pieces of one new row's K and V
  for (;;) {
    if (tid == 0) sm.item = atomicAdd(mctr, 1u);
    lds_sync();
    const uint32_t rel = __builtin_amdgcn_readfirstlane(sm.item);
    lds_sync();
    if (rel >= count) {
      if (tid == 0 && rel == count + wgs - 1u) __hip_atomic_store(mctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    if (STORE && rel < nstore) {
      // Rows [4g, 4g + 4).
      const int64_t t0 = STORE_ROWS * (list + (int)rel * nlist);
      store_new_rows<FP8>(p, t0 * per_tok, min((int64_t)p.nnew, t0 + STORE_ROWS) * per_tok, tid);
      continue;
    }
    const int task = list + (int)(rel - nstore) * nlist;
    const int b = task / p.hkv, h = task % p.hkv;
    const int L = min(max(p.dlens[b], 0), p.dtab_width * p.block_size);
    const uint32_t nch = (uint32_t)max(1, (L + dchunk - 1) / dchunk);
    if (nch == 1) continue;
    uint32_t* ticket = reinterpret_cast<uint32_t*>(&p.counters[b * p.hkv + h]);
    if (tid == 0) {
      const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
      bool ok = true;
      while (__hip_atomic_load(ticket, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < nch) {
        if ((int64_t)(__builtin_amdgcn_s_memrealtime() - t0) > p.merge_wait_ticks) {
          ok = false;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      if (!ok) {
        // The chunks did not all arrive in time (workgroups of this launch
        // could not run: the GPU is shared, or the grid exceeds what it
        // holds).  No merge: the outputs of (b, h) are set to NaN below and
        // the event counter reports it to the host.  The ticket still drops
        // by nch, so the late increments bring it back to zero.
        __hip_atomic_fetch_add(reinterpret_cast<uint32_t*>(p.ctrl) + EVENTS_OFFSET / 4 + EV_MERGE_GAVE_UP, 1u,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_add(ticket, 0u - nch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      sm.row = ok ? 1 : 0;
    }
    lds_sync();
    const bool mine = __builtin_amdgcn_readfirstlane(sm.row) != 0;
    lds_sync();
    if (mine) {
      decode_final(p, b, h, sm.off[p.np + b] - decode_base + h, (int)nch, tid);
    } else {
      // NaN (bf16 0x7fc0) in every output of (b, h), so a consumer that does
      // not check the workspace sees invalid values rather than stale ones.
      for (int u = tid; u < p.G * (HD / 2); u += NT) {
        const int hn = u / (HD / 2), d = 2 * (u % (HD / 2));
        *reinterpret_cast<uint32_t*>(p.out + (int64_t)b * p.out_stride + (int64_t)(h * p.G + hn) * HD + d) =
            0x7fc07fc0u;
      }
    }
  }
}

// s_waitcnt vmcnt(base + extra) for a small runtime `extra` (0..7).
template <int BASE>
__device__ __forceinline__ void wait_vm(int extra) {
  switch (extra) {
    case 0: __builtin_amdgcn_s_waitcnt(vmcnt_imm(BASE)); break;
    case 1: __builtin_amdgcn_s_waitcnt(vmcnt_imm(BASE + 1)); break;
    case 2: __builtin_amdgcn_s_waitcnt(vmcnt_imm(BASE + 2)); break;
    case 3: __builtin_amdgcn_s_waitcnt(vmcnt_imm(BASE + 3)); break;
    case 4: __builtin_amdgcn_s_waitcnt(vmcnt_imm(BASE + 4)); break;
    case 5: __builtin_amdgcn_s_waitcnt(vmcnt_imm(BASE + 5)); break;
    case 6: __builtin_amdgcn_s_waitcnt(vmcnt_imm(BASE + 6)); break;
    default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(BASE + 7)); break;
  }
}

// Runs this workgroup's remaining items, all decode items, starting with
// relative index rel0 (row r0), and returns with sm.item holding the last
// in-list or out-of-list fetch result.  Every fetch issued is consumed, and
// none is issued after an out-of-list one (later ones add 0).
//
// Vector memory operations of item k (cur), in issue order; G = step loads per
// wavefront, H = merge stores per wavefront, [0] = wavefront 0 only:
//   step 0: step (cur, 2)
//   step 1: [0] ticket of prev   [0] metadata of nxt   step (cur, 3)
//   step 2: Q(nxt)   step (nxt, 0)
//   step 3: merge stores (H)   step (nxt, 1)   [0] fetch of the item after nxt
// so the waits before steps 0..3 allow H+G+[1], G, G, G+1 younger operations.
// nxt is learned at step 1 from the fetch issued at the end of the previous
// item, so a workgroup holds at most its current item and one claimed item
// that has not started.
template <bool FP8, bool FOLD, bool NT>
__device__ void decode_run(const Params& p, Smem& sm, uint8_t* st0, uint8_t* st1, uint8_t* qbuf, int list, int nlist,
                           uint32_t count, uint32_t base, uint32_t* ctr, int decode_base, int nrows, uint32_t rel0,
                           int r0, int dchunk, int tid) {
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  const bool w0 = wave == 0;
  const bool half = dchunk < d_chunk<FP8>();  // steps 2 and 3 of every item are empty
  uint8_t* sa = st0 + wave * WSTAGE;  // even steps
  uint8_t* sb = st1 + wave * WSTAGE;  // odd steps
  float* ca = sm.u.dec.sc[0][wave];   // E4M3FN scales of even and odd steps
  float* cb = sm.u.dec.sc[1][wave];
  // E4M3FN with the KV write folded in: the row's new K and V rows of even
  // and odd steps, in the Q buffer past the item's Q (at most 8 query heads
  // per kv head, checked on the host).
  uint8_t* na = qbuf + 2048 + wave * 512;
  uint8_t* nb = qbuf + QBUF + 2048 + wave * 512;
  auto tnew_of = [&](const DMeta& mm, int s) {
    return decode_L(p, mm) - 1 - (mm.tok0 + s * d_step<FP8>() + wave * d_dt<FP8>());
  };
  constexpr int GROUP = d_group<FP8, FOLD>();
  const int hgp = (p.G + 3) >> 2;  // merge stores per wavefront and item
  auto item_of = [&](uint32_t rel) { return decode_base + dec_index(list, nlist, FP8 ? p.hkv : 1, (int)rel); };

  // Prologue: the first item's metadata, then the same operations the
  // loop's last step leaves in flight (with stand-in stores for the merge).
  const bool rot = sm.drot;
  DMeta cur = decode_geom(p, r0, __builtin_amdgcn_readfirstlane(item_of(rel0) - sm.off[r0]), item_of(rel0), decode_base,
                          dchunk, rot);
  if (w0) decode_meta_dma<FP8>(p, sm, cur, 0, lane);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  lds_sync();
  decode_meta_read<FP8>(cur, sm, 0, wave);
  decode_issue_q(p, qbuf, cur, wave, lane);
  decode_issue<FP8, FOLD, NT>(p, sa, ca, na, cur, 0, wave, lane);
  for (int i = 0; i < hgp; ++i)
    if (lane < 33) store16(reinterpret_cast<uint8_t*>(p.ctrl) + TRASH_OFFSET + 16 * lane, u32x4{0, 0, 0, 0});
  decode_issue<FP8, FOLD, NT>(p, sb, cb, nb, cur, 1, wave, lane);
  uint32_t f = 0;
  bool fetching = true;  // the fetch in flight is a real one
  if (tid == 0) f = atomic_add_ret(ctr, 1u);

  DMeta prev = cur;
  bool due = false;  // prev's partial is stored and its ticket not yet taken
  for (int k = 0;; ++k) {
    const uint8_t* qcur = qbuf + (k & 1) * QBUF;
    uint8_t* qnxt = qbuf + ((k + 1) & 1) * QBUF;

    // Step 0: (cur, 0) and Q(cur) have landed.
    wait_vm<GROUP>(hgp + (w0 ? 1 : 0));
    lds_sync();
    u32x4 qv[4];
    {
      const int hn = min(n, p.G - 1);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) qv[kk] = ld16(qcur + hn * ROWB + 16 * (4 * kk + g));
    }
    f32x4 o[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt] = f32x4{0, 0, 0, 0};
    float m = NEG_INF, l = 0.0f;
    decode_wstep<FP8, FOLD>(p, sa, ca, na, decode_ntok<FP8>(p, cur, 0, wave), tnew_of(cur, 0), qv, o, m, l, lane);
    decode_issue<FP8, FOLD, NT>(p, sa, ca, na, cur, 2, wave, lane);

    // Step 1: (cur, 1) has landed, and with it prev's stores (every
    // wavefront's, after the barrier) and the fetch.  Wavefront 0 finds the
    // fetched item's row, broadcasts it and loads the item's metadata.
    wait_vm<GROUP>(0);
    lds_sync();
    if (tid == 0) atomic_add_noret(&p.counters[prev.b * p.hkv + prev.h], due ? 1u : 0u);
    due = false;
    bool has1 = false;
    DMeta nxt = cur;
    if (w0) {
      if (fetching) {
        const uint32_t rel1 = __builtin_amdgcn_readfirstlane(after_wait(f)) - base;
        has1 = rel1 < count;
        if (has1) {
          const int item = item_of(rel1);
          const int r = find_row(sm, item, p.np, nrows, lane);
          const int local = __builtin_amdgcn_readfirstlane(item - sm.off[r]);
          nxt = decode_geom(p, r, local, item, decode_base, dchunk, rot);
          if (tid == 0) {
            sm.bcast[0] = r;
            sm.bcast[1] = local;
          }
        }
        if (tid == 0) sm.item = rel1;
      }
      decode_meta_dma<FP8>(p, sm, nxt, (k + 1) & 1, lane);
    }
    decode_wstep<FP8, FOLD>(p, sb, cb, nb, decode_ntok<FP8>(p, cur, 1, wave), tnew_of(cur, 1), qv, o, m, l, lane);
    decode_issue<FP8, FOLD, NT>(p, sb, cb, nb, cur, 3, wave, lane);

    // Step 2: (cur, 2) and nxt's metadata have landed; the broadcast is
    // visible after the barrier.
    wait_vm<GROUP>(0);
    lds_sync();
    if (fetching) {
      const uint32_t rel1 = __builtin_amdgcn_readfirstlane(sm.item);
      has1 = rel1 < count;
      if (has1) {
        if (!w0)
          nxt = decode_geom(p, __builtin_amdgcn_readfirstlane(sm.bcast[0]),
                            __builtin_amdgcn_readfirstlane(sm.bcast[1]), item_of(rel1), decode_base, dchunk, rot);
        decode_meta_read<FP8>(nxt, sm, (k + 1) & 1, wave);
      }
    }
    if (!has1) nxt = cur;  // no next item: its loads repeat the current item's
    decode_issue_q(p, qnxt, nxt, wave, lane);
    if (!half)
      decode_wstep<FP8, FOLD>(p, sa, ca, na, decode_ntok<FP8>(p, cur, 2, wave), tnew_of(cur, 2), qv, o, m, l, lane);
    decode_issue<FP8, FOLD, NT>(p, sa, ca, na, nxt, 0, wave, lane);

    // Step 3: (cur, 3) has landed.
    wait_vm<GROUP + 1>(0);
    if (!half)
      decode_wstep<FP8, FOLD>(p, sb, cb, nb, decode_ntok<FP8>(p, cur, 3, wave), tnew_of(cur, 3), qv, o, m, l, lane);
    lds_sync();  // every wavefront's last step is done: merge area and stage-1 regions are free
    decode_merge(p, sm, st1, cur, tid, o, m, l);
    decode_issue<FP8, FOLD, NT>(p, sb, cb, nb, nxt, 1, wave, lane);
    fetching = fetching && has1;
    if (tid == 0) f = atomic_add_ret(ctr, fetching ? 1u : 0u);
    prev = cur;
    due = decode_nch(p, cur) > 1;
    if (!has1) break;
    cur = nxt;
  }
  // The last item's stores (and the repeated loads) complete here.
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  lds_sync();
  if (tid == 0 && due) atomic_add_noret(&p.counters[prev.b * p.hkv + prev.h], 1u);
}

// ------------------------------------------------------------ direct decode
// One chunk of a direct launch: nrun steps of item m (its block-table entries
// at `entries`: one per step, E4M3FN one per step and wavefront), two in
// flight, then the cross-wavefront merge and, with several chunks in the
// row, the split-K merge by the chunk whose ticket increment arrives last
// (records of chunk c of (row, head) at dfirst + c * hkv).  mid() runs once
// after the first steps' loads are issued; it returns whether it issued
// memory operations of its own (the first wait then covers everything).
// Ends with LDS free for the next chunk.
template <bool FP8, bool FOLD, typename Mid>
__device__ __forceinline__ void run_chunk(const Params& p, Smem& sm, uint8_t* stage0, uint8_t* stage1, uint8_t* qbuf,
                                          const int* entries, const DMeta& m, int nrun, int nch, int dfirst, int tid,
                                          Mid&& mid) {
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Step s as an item of one step (its first token, block and span), for the
  // decode helpers.
  auto step = [&](int s) {
    DMeta ms = m;
    ms.tok0 = m.tok0 + s * d_step<FP8>();
    ms.span = d_step<FP8>();
    ms.page[0] = __builtin_amdgcn_readfirstlane(entries[FP8 ? 4 * s + wave : s]);
    return ms;
  };

  // Steps alternate between the two stages, two in flight; every stage and
  // its scales and new rows are private to the wavefront, so a step needs
  // only its loads' wait (GROUP vector memory operations per step and
  // wavefront).
  constexpr int GROUP = d_group<FP8, FOLD>();
  uint8_t* sa = stage0 + wave * WSTAGE;
  uint8_t* sb = stage1 + wave * WSTAGE;
  float* ca = sm.u.dec.sc[0][wave];
  float* cb = sm.u.dec.sc[1][wave];
  uint8_t* na = qbuf + 2048 + wave * 512;
  uint8_t* nb = qbuf + QBUF + 2048 + wave * 512;
  decode_issue<FP8, FOLD>(p, sa, ca, na, step(0), 0, wave, lane);
  if (nrun > 1) decode_issue<FP8, FOLD>(p, sb, cb, nb, step(1), 0, wave, lane);
  const bool side = mid();
  const int n = lane & 15, g = lane >> 4;
  u32x4 qv[4];
  {
    const int hn = min(n, p.G - 1);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) qv[kk] = ld16(qbuf + hn * ROWB + 16 * (4 * kk + g));
  }
  f32x4 o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = f32x4{0, 0, 0, 0};
  float mx = NEG_INF, l = 0.0f;
  const int L = decode_L(p, m);
  for (int s = 0; s < nrun; ++s) {
    const bool odd = s & 1;
    if (s + 1 < nrun && !(s == 0 && side)) __builtin_amdgcn_s_waitcnt(vmcnt_imm(GROUP));
    else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    const DMeta ms = step(s);
    decode_wstep<FP8, FOLD>(p, odd ? sb : sa, odd ? cb : ca, odd ? nb : na, decode_ntok<FP8>(p, ms, 0, wave),
                            L - 1 - (ms.tok0 + wave * d_dt<FP8>()), qv, o, mx, l, lane);
    if (s + 2 < nrun) decode_issue<FP8, FOLD>(p, odd ? sb : sa, odd ? cb : ca, odd ? nb : na, step(s + 2), 0, wave, lane);
  }
  lds_sync();
  decode_merge(p, sm, stage1, m, tid, o, mx, l);
  if (nch > 1) {
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // this workgroup's records stored before its ticket
    __syncthreads();
    if (tid == 0) {
      const uint32_t old = atomic_add_ret(&p.counters[m.b * p.hkv + m.h], 1u);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
      sm.row = (int)after_wait(old) == nch - 1 ? 1 : 0;
    }
    __syncthreads();
    if (sm.row) decode_final(p, m.b, m.h, dfirst, nch, tid);
  }
  __syncthreads();
}


constexpr int DIRECT_ENTRIES = 32;  // block-table entries of a direct chunk (at most 1024 tokens)
// Short decode-only launches: one workgroup per (row, chunk, kv head), no work
// lists, no prologue over the batch.  Chunks are `ns` workgroup steps (two
// in flight), up to 1024 tokens; the grid covers every chunk the tables can
// hold (chunks past a row's length exit after reading its length), so it is
// sized from shapes only.  Workgroup x takes kv head (x / 8) % hkv of group
// g = j * 8 + (x + j) % 8, j = x / (8 hkv): the kv heads of one (row, chunk)
// run on one XCD (x % 8), where they share the lines of the E4M3FN scale
// rows; groups g = c * nd + b put every row's first chunks at the front of
// the grid, and the rotation by j spreads a row's chunks over the XCDs (with
// nd a multiple of 8, x % 8 alone would put every chunk of a row on one XCD:
// 24 rows of 256-4096 tokens, 50.3 -> 45.5 us).
// A row with several chunks merges them in the workgroup whose ticket
// increment arrives last (records stored before the increment, merged in
// chunk order, so the result does not depend on which one merges); the
// launch leaves every ticket at zero.  With the KV write folded in, the first
// workgroups also copy the new rows to their slots (nothing in the launch
// reads those slots: a decode row's newest token comes from its new row).
template <bool FP8, bool FOLD>
__global__ void __launch_bounds__(NT, 2) decode_direct_kernel(Params p, int nch_cap, int ns, int spread) {
  __shared__ Smem sm;
  __shared__ int dmeta[1 + DIRECT_ENTRIES];  // row length, then the chunk's block-table entries
  __shared__ __attribute__((aligned(16))) uint8_t stage0[4 * WSTAGE];
  __shared__ __attribute__((aligned(16))) uint8_t stage1[4 * WSTAGE];
  __shared__ __attribute__((aligned(16))) uint8_t qbuf[2 * QBUF];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int x = blockIdx.x;

  // Once per workgroup, on every path (after the item's loads are issued
  // where it has one): its share of the KV write (4 * NT pieces per
  // workgroup) and of the zeros for query rows past every decode and prefill
  // row.
  auto side_work = [&]() {
    bool any = false;
    if constexpr (FOLD) {
      const int64_t per_wg = 4 * NT, all = (int64_t)p.nnew * (2 * (p.hkv * HD / 8));
      if ((int64_t)x * per_wg < all) {
        store_new_rows<FP8>(p, (int64_t)x * per_wg, min(all, (int64_t)(x + 1) * per_wg), tid);
        any = true;
      }
    }
    const int64_t covered = (int64_t)p.q_off_prefill + (p.np_all > 0 ? max(p.cu_q_all[p.np_all], 0) : 0);
    if (covered < p.num_q_rows) {
      any = true;
      const int per_row = p.hkv * p.G * HD / 8;
      const int64_t pieces = (p.num_q_rows - covered) * per_row;
      for (int64_t i = (int64_t)x * NT + tid; i < pieces; i += (int64_t)gridDim.x * NT) {
        const int64_t row = covered + i / per_row;
        *reinterpret_cast<u32x4*>(p.out + row * p.out_stride + 8 * (i % per_row)) = u32x4{0, 0, 0, 0};
      }
    }
    return any;
  };

  // With `spread` (bf16 pools, kv heads a multiple of the 8 XCDs, at most
  // two rounds of workgroups) the kv heads of a group are consecutive
  // workgroups instead, on different XCDs: XCD k reads kv heads k, k + 8, ...
  // of every group, each 256-byte slice of a 2 KiB pool row at about the time
  // the other XCDs read the row's other slices (24 rows of 256-4096 tokens
  // 45.4 -> 43.9 us; 16 rows of 64-1,024 14.9 -> 14.7 us).  Longer launches,
  // whose rounds drift apart, and fewer kv heads keep the mapping above (64
  // rows of 512-4096 tokens measured 125.2 -> 128.1 us spread, 24 rows at 4
  // kv heads 26.8 -> 31.6 us).
  const bool spr = !FP8 && spread;
  const int jx = x / (8 * p.hkv);
  const int grp = spr ? x / p.hkv : jx * 8 + (x + jx) % 8;
  if (grp >= nch_cap * p.nd) {
    side_work();
    return;
  }
  DMeta m;
  m.c = grp / p.nd;
  m.b = grp % p.nd;
  m.h = spr ? x % p.hkv : (x / 8) % p.hkv;
  m.dindex = (m.b * nch_cap + m.c) * p.hkv + m.h;
  m.span = ns * d_step<FP8>();
  m.tok0 = m.c * m.span;
  // The row's length and the chunk's block-table entries (bf16: one per
  // workgroup step; E4M3FN: one per step and wavefront, since a 128-token
  // step may span two blocks of 64), and Q (it depends on the row and head
  // only), in one round trip.
  {
    constexpr int PER = FP8 ? 4 : 1;
    const int e = lane - 1;
    const int tok = m.tok0 + (e / PER) * d_step<FP8>() + (e % PER) * d_dt<FP8>();
    const int32_t* src = (e >= 0 && e < PER * ns)
                             ? p.dtab + (int64_t)m.b * p.dtab_stride + min(tok / p.block_size, p.dtab_width - 1)
                             : p.dlens + m.b;
    if (wave == 0 && lane <= PER * ns) dma4(src, lds_addr(dmeta));
  }
  decode_issue_q(p, qbuf, m, wave, lane);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  __syncthreads();
  m.len = __builtin_amdgcn_readfirstlane(dmeta[0]);
  const int nch = decode_nch(p, m);
  if (m.c >= nch) {
    side_work();
    return;
  }
  // Steps past the row's end are not run.
  const int nrun = max(1, min(ns, (decode_L(p, m) - m.tok0 + d_step<FP8>() - 1) / d_step<FP8>()));
  run_chunk<FP8, FOLD>(p, sm, stage0, stage1, qbuf, dmeta + 1, m, nrun, nch, m.b * nch_cap * p.hkv + m.h, tid,
                       side_work);
}

// --------------------------------------------------------------- prefill item
// SPLITK (prefill-only launches): with `split`, the row's items come in
// pairs that cover the first and the second half of each block's key tiles
// (local index ((block * 2 + part) * hkv + h) * HG + hg, global `item`); each
// writes (O, m, l) of its range as a record, and the one that arrives second
// on the pair's ticket merges both and writes the output.
template <bool FP8, int NQT, bool FOLD, bool SPLITK = false>
__device__ void prefill_item(const Params& p, Smem& sm, uint8_t* st0, uint8_t* st1, int r, int local, int tid,
                             int item = 0, bool split = false) {
  static_assert(!(FP8 && FOLD), "E4M3FN launches with prefill rows run the store kernel first");
  constexpr int BQ = 16 * NQT;
  const int lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const bool two = SPLITK && split;
  const int hg = local % p.HG;
  const int t = local / p.HG;
  const int h = t % p.hkv;
  const int u = t / p.hkv;
  const int part = two ? u & 1 : 0;
  const int qb_rev = two ? u >> 1 : u;

  const PfRow geo = pf_row(p, r);
  const int q_start = geo.q_start, Lq = geo.Lq, k_start = geo.k_start, Lk = geo.Lk;
  const int prefix = geo.prefix;  // bottom-right causal alignment
  const bool paged = p.ptab != nullptr;

  const int nqb = (Lq + BQ - 1) / BQ;
  const int q0 = (nqb - 1 - qb_rev) * BQ;  // heaviest blocks are pulled first
  // An item past the row's blocks (its count and block size disagree) reads
  // and writes nothing.
  if (q0 < 0) return;
  const int qend = min(q0 + BQ, Lq);
  const int kend = min(Lk, max(0, prefix + qend));
  // Key range of this item: all tiles, or one half (the first half takes the
  // extra tile of an odd count; the second holds the causal boundary).
  const int tcut = (kend + 2 * TT - 1) / (2 * TT);
  const int kstart = two && part ? tcut * TT : 0;
  const int kstop = two && !part ? min(kend, tcut * TT) : kend;
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
  // tile is in flight while the current one is consumed.  E4M3FN pool bytes
  // take the same route into the second half of the next tile's buffer (K
  // codes, then V codes, 8 KiB each, 16-byte chunk c of row r in slot
  // c ^ (r & 7)) and their scales straight to sm.u.pf.ks/vs; the MFMA
  // operands are converted from the codes where they are read.  Rows past the
  // valid keys are zero (bf16) or masked where read (codes).
  const int* prow = p.ptab + (int64_t)r * p.ptab_stride;
  const int npages = paged ? (kend + p.block_size - 1) / p.block_size : 0;
  const bool cached = npages <= MAX_PAGES;
  typedef __attribute__((address_space(3))) const int lds_int;
  lds_int* pages = (lds_int*)(sm.u.pf.pages);
  // Lane-constant element offsets of this thread's 4 tile rows (row
  // 16 wave + 4 it + lane / 16, swizzled 16-byte chunk) from the tile's first
  // key, lowered by 1024 it bytes: a wavefront's four K (or V) loads of a full
  // tile fill 4 KiB of LDS and share one M0 write, each adding its 1024 it
  // as the instruction offset (rows are at least 128 elements apart, checked
  // on the host, so the offsets stay non-negative).
  const int krow = paged ? p.hkv * HD : (int)p.k_stride;  // row strides < 2^25 elements (checked on the host)
  const int vrow = paged ? p.hkv * HD : (int)p.v_stride;
  // FOLD: elements; otherwise bytes (row strides < 2^25 elements: 63 rows
  // stay below 2^32 bytes), for the SGPR-base loads of issue_tile.
  int kgo[4], vgo[4];
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int row = 16 * wave + 4 * it + (lane >> 4);
    kgo[it] = (FOLD ? 1 : 2) * (row * krow + 8 * ((tid & 15) ^ (row & 15)) - 512 * it);
    vgo[it] = (FOLD ? 1 : 2) * (row * vrow + 8 * ((tid & 15) ^ ((row & 7) << 1)) - 512 * it);
  }
  // Tiles per KV block as a multiplicative inverse (ceil(2^32 / tiles), exact
  // for tile indices below 2^16 and 2 to 2^16 tiles per block; one tile per
  // block, whose inverse 2^32 does not fit, is taken apart), and the element
  // strides of a block and a pool row.
  const uint32_t tpb = (uint32_t)(p.block_size / TT);
  const uint32_t tpb_inv = (uint32_t)((0xffffffffull + tpb) / tpb);
  const int row_el = p.hkv * HD;
  const int64_t blk_el = (int64_t)p.block_size * row_el;
  auto issue_tile = [&](int kv0, int buf) -> int {
    const int ntok = min(TT, kend - kv0);
    bool ok = true;
    int64_t slot0 = 0, kbase, vbase;  // element offsets of the tile's first key, head h
    if (paged && FOLD && kv0 < TT * 65536) {
      // The folded instantiation, short of SGPRs, finds the block without a
      // division (24 decode rows of 256-4096 tokens and two 512-token chunks:
      // 68.0 -> 67.4 us; the other instantiations ran slower this way).
      const uint32_t t = (uint32_t)kv0 / TT;
      const int bi = tpb == 1 ? (int)t : (int)__umulhi(t, tpb_inv);  // t / tiles per block
      const int page = cached ? pages[bi] : prow[bi];
      ok = page >= 0 && page < p.num_blocks;
      const int off = kv0 - bi * p.block_size;
      slot0 = ok ? (int64_t)page * p.block_size + off : 0;
      kbase = vbase = ok ? (int64_t)page * blk_el + (int64_t)(off * row_el + h * HD) : (int64_t)h * HD;
    } else if (paged) {
      const int page = cached ? pages[kv0 / p.block_size] : prow[kv0 / p.block_size];
      ok = page >= 0 && page < p.num_blocks;
      slot0 = ok ? (int64_t)page * p.block_size + kv0 % p.block_size : 0;
      kbase = vbase = slot0 * p.hkv * HD + (int64_t)h * HD;
    } else {
      kbase = (int64_t)(k_start + kv0) * p.k_stride + (int64_t)h * HD;
      vbase = (int64_t)(k_start + kv0) * p.v_stride + (int64_t)h * HD;
    }
    // With the KV write in this launch (FOLD, contiguous new rows of the pool's
    // row length), tiles from the prefix on hold only new tokens: they are read
    // from the new rows (key j: new row qrow0 + j - prefix), whose slots this
    // launch writes at its end.  The row offsets are the pool's.  (The tile
    // that straddles the prefix, if any, was written to the pool by this item
    // before its first tile.)
    bool fresh = false;
    if constexpr (FOLD) fresh = paged && kv0 >= prefix && qrow0 - prefix + kv0 + ntok <= p.nnew;
    if (fresh) ok = true;
    const int nv = ok ? ntok : 0;
    if (src_fp8 && !fresh) {
      // The codes stay codes: K and V code rows (128 bytes, 16-byte chunk c
      // of row r at slot c ^ (r & 7)) go to the second half of the buffer and
      // the MFMA operands are converted from them as they are read.  All 64
      // rows of the tile's block are loaded (they lie in that block,
      // block_size being a multiple of 64); rows past the valid keys are
      // masked where they are read.  Without a valid block the codes and
      // scales are zeros (keys of score 0 and value 0).
      uint8_t* stg = (buf ? st1 : st0) + TILE_BYTES;
      if (!ok) {
#pragma unroll
        for (int it = 0; it < 4; ++it) st16(stg + 16 * (it * NT + tid), u32x4{0, 0, 0, 0});
        if (tid < TT) {
          sm.u.pf.ks[buf][tid] = 0.0f;
          sm.u.pf.vs[buf][tid] = 0.0f;
        }
        return nv;
      }
      const uint8_t* kc = static_cast<const uint8_t*>(p.k_cache) + kbase;
      const uint8_t* vc = static_cast<const uint8_t*>(p.v_cache) + vbase;
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const int q = it * NT + tid;  // 16-byte slot q: row q >> 3, slot q & 7
        const int off = (q >> 3) * krow + 16 * ((q & 7) ^ ((q >> 3) & 7));
        const uint32_t dst = lds_addr(stg + 16 * (it * NT + wave * 64));
        dma16(kc + off, dst);
        dma16(vc + off, dst + 8192);
      }
      if (wave < 2) {
        const float* sc = wave ? p.v_scale : p.k_scale;
        dma4(sc + (slot0 + lane) * p.hkv + h, lds_addr(wave ? sm.u.pf.vs[buf] : sm.u.pf.ks[buf]));
      }
      return nv;
    }
    const int ret = nv;
    const uint16_t* ksrc = (paged ? static_cast<const uint16_t*>(p.k_cache) : p.k) + kbase;
    const uint16_t* vsrc = (paged ? static_cast<const uint16_t*>(p.v_cache) : p.v) + vbase;
    if (fresh) {
      const int64_t t0 = (qrow0 - prefix + kv0) * p.nk_stride + (int64_t)h * HD;
      ksrc = p.nk + t0;
      vsrc = p.nv + t0;
    }
    // Inline-asm DMA: the compiler does not track these loads, so it inserts
    // no wait for them before the current tile's LDS reads (it cannot tell
    // which buffer a DMA writes); the loop waits for them explicitly.
    const uint32_t kdst = lds_addr((buf ? st1 : st0) + 16 * wave * ROWB);
    const uint32_t vdst = kdst + TILE_BYTES;
    // Without the folded KV write the tile base goes to SGPRs and each load
    // adds a 32-bit lane offset (four cold 1.1k-token prefill rows: 105 -> 101
    // us); the folded instantiation, short of SGPRs, keeps 64-bit lane
    // addresses (its launch ran 1% slower with SGPR bases).
    const void* kb = FOLD ? nullptr : uniform_ptr(ksrc);
    const void* vb = FOLD ? nullptr : uniform_ptr(vsrc);
    auto dma_k = [&](int it) {
      if constexpr (FOLD) dma16(ksrc + kgo[it] + 512 * it, kdst + 4 * it * ROWB);
      else dma16_at(kb, (uint32_t)(kgo[it] + 1024 * it), kdst + 4 * it * ROWB);
    };
    auto dma_v = [&](int it) {
      if constexpr (FOLD) dma16(vsrc + vgo[it] + 512 * it, vdst + 4 * it * ROWB);
      else dma16_at(vb, (uint32_t)(vgo[it] + 1024 * it), vdst + 4 * it * ROWB);
    };
    if (nv == TT) {  // full tile: DMA only
      if constexpr (FOLD) {
        dma16x4(ksrc + kgo[0], ksrc + kgo[1], ksrc + kgo[2], ksrc + kgo[3], kdst);
        dma16x4(vsrc + vgo[0], vsrc + vgo[1], vsrc + vgo[2], vsrc + vgo[3], vdst);
      } else if constexpr (!FP8) {
        dma16x4_at(kb, kgo, kdst);
        dma16x4_at(vb, vgo, vdst);
      } else {
        // (The E4M3FN instantiations, at 256 VGPRs, spilled with the four
        // offsets live at once.)
#pragma unroll
        for (int it = 0; it < 4; ++it) {
          dma_k(it);
          dma_v(it);
        }
      }
      return ret;
    }
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int row = 16 * wave + 4 * it + (lane >> 4);
      if (row < nv) {
        dma_k(it);
        dma_v(it);
      } else {
        st16((buf ? st1 : st0) + row * ROWB + ((tid & 15) << 4), u32x4{0, 0, 0, 0});
        st16((buf ? st1 : st0) + TILE_BYTES + row * ROWB + ((tid & 15) << 4), u32x4{0, 0, 0, 0});
      }
    }
    return ret;
  };
  // After the tile of buffer `buf` is issued: tiles of bf16 rows in an
  // E4M3FN launch take unit scales; tiles of E4M3FN codes need nothing (their
  // operands are converted where they are read).
  auto commit_tile = [&](int buf, int nv, int kv0) {
    if (!src_fp8) {
      // bf16 rows of an E4M3FN launch: unit scales (read after the next
      // tile's barrier).
      if (FP8 && tid < TT) {
        sm.u.pf.ks[buf][tid] = 1.0f;
        sm.u.pf.vs[buf][tid] = 1.0f;
      }
      return;
    }
  };

  // Lane-constant LDS byte offsets of the MFMA operands within a tile: K rows
  // 16mt+n (mt added per use), V^T rows 32ks + 4g + n/4 (+16 for slots 4-7).
  int koff[4], voff[8];
#pragma unroll
  for (int st = 0; st < 4; ++st) koff[st] = k_off(n, 4 * st + g);
  // Code tiles (E4M3FN): K code row r at 128 r with 16-byte chunk c in slot
  // c ^ (r & 7) (K fragment reads: row n of each 16-row block, chunk
  // 2 (jj >> 1) + g / 2, bytes 8 (g & 1)); the V^T reads pass row j = n / 2
  // of an 8-row block (key 4g + j, or 16 + 4g + j - 4), bytes 8 (n & 1).
  int kcoff[4] = {0, 0, 0, 0}, vcoff = 0, vcsw = 0;
  if constexpr (FP8) {
#pragma unroll
    for (int st = 0; st < 4; ++st) kcoff[st] = n * 128 + 16 * ((2 * st + (g >> 1)) ^ (n & 7)) + 8 * (g & 1);
    const int vkey = (n >> 1) < 4 ? 4 * g + (n >> 1) : 12 + 4 * g + (n >> 1);
    vcoff = vkey * 128 + 8 * (n & 1);
    vcsw = vkey & 7;
  }
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) voff[dt] = v_off(4 * g + (n >> 2), 2 * dt + ((n & 3) >> 1)) + ((n & 1) << 3);

  // The row's block table goes to LDS once, so no tile waits on a table load.
  if (cached)
    for (int i = tid; i < npages; i += NT) sm.u.pf.pages[i] = prow[i];
  __syncthreads();
  if constexpr (FOLD) {
    // The tile that straddles the prefix reads its keys from the pool, so this
    // item first writes that tile's new tokens (head h) to their slots itself:
    // every item reading the tile writes the same bytes before reading them.
    const int s0 = prefix & ~(TT - 1), s1 = min(kend, s0 + TT);
    if (paged && (prefix & (TT - 1)) && prefix < s1) {
      const int n_new = s1 - prefix;  // tokens, each 16 + 16 pieces of 16 bytes (K, V of head h)
      for (int i = tid; i < 32 * n_new; i += NT) {
        const int jj = prefix + (i >> 5), pc = i & 15;
        const bool isv = i & 16;
        const int64_t t = min(qrow0 + jj - prefix, (int64_t)p.nnew - 1);
        const int page = cached ? pages[jj / p.block_size] : prow[jj / p.block_size];
        if (page < 0 || page >= p.num_blocks) continue;
        const int64_t slot = (int64_t)page * p.block_size + jj % p.block_size;
        const uint16_t* src = (isv ? p.nv + t * p.nv_stride : p.nk + t * p.nk_stride) + (int64_t)h * HD + 8 * pc;
        const int64_t e = slot * p.hkv * HD + (int64_t)h * HD + 8 * pc;
        uint16_t* dst = static_cast<uint16_t*>(const_cast<void*>(isv ? p.v_cache : p.k_cache)) + e;
        *reinterpret_cast<u32x4*>(dst) = ld16(src);
      }
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // written before any DMA of this item reads them
      __syncthreads();
    }
  }
  if (kstart < kstop) {
    const int nv0 = issue_tile(kstart, 0);
    commit_tile(0, nv0, kstart);
  }
  // Each tile is processed as two halves of 32 keys,
  // software-pipelined so that MFMA work of one half and the softmax VALU
  // work of the other are independent and can be interleaved:
  //   QK(h0);  QK(h1) | softmax(h0);  [rescale];  PV(h0) | softmax(h1);
  //   [rescale];  PV(h1).
  // The rescale of O (rare with the lazy offset) sits between the regions.
  // Interior tiles (no key past the valid rows or the causal edge) run in a
  // loop of their own without masking code.
  auto tile = [&](auto mask_tag, auto codes_tag, int kv0, int j) {
    constexpr bool MASK = decltype(mask_tag)::value;
    constexpr bool CODES = decltype(codes_tag)::value;  // E4M3FN codes in the buffer's second half
    const int buf = j & 1;
    const int ntok = min(TT, kend - kv0);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    lds_sync();
    const bool more = kv0 + TT < kstop;
    const uint8_t* kt = buf ? st1 : st0;
    const uint8_t* vt = kt + TILE_BYTES;
    // Boundary tiles of codes: byte j of a V^T read is key kperm(j) of the
    // half (keys 4g + j, then 16 + 4g + j - 4); kept when below ntok.
    uint64_t keep0 = ~0ull, keep1 = ~0ull;
    if constexpr (CODES && MASK) {
      keep0 = keep1 = 0;
#pragma unroll
      for (int jb = 0; jb < 8; ++jb) {
        const int key = (jb < 4 ? 4 * g + jb : 12 + 4 * g + jb);
        keep0 |= (key < ntok ? 0xffull : 0ull) << (8 * jb);
        keep1 |= (32 + key < ntok ? 0xffull : 0ull) << (8 * jb);
      }
    }
    // K fragment jj of half h: rows 16*(2h + (jj & 1)) + n, k-step jj >> 1
    // (from codes: the 8 bytes of d = 32 (jj >> 1) + 8g.. of that row).
    auto kread_h = [&](int h, int jj) -> u32x4 {
      if constexpr (CODES) return fp8x8_to_bf16x8(ld8(vt + (2 * h + (jj & 1)) * 16 * 128 + kcoff[jj >> 1]));
      else return ld16(kt + (2 * h + (jj & 1)) * 16 * ROWB + koff[jj >> 1]);
    };
    auto vread = [&](int i) -> bf16x8 {  // V^T operand: k-step (half) i >> 3, d-tile i & 7
      if constexpr (CODES) {
        // Transposed byte read of the 8 keys of this lane's operand slots
        // (d = 16 (i & 7) + n); codes of keys past the valid ones (NaN
        // patterns possible) are zeroed in boundary tiles.
        u32x2 c = lds_tr8(vt + 8192 + (i >> 3) * 32 * 128 + vcoff + 16 * ((i & 7) ^ vcsw));
        if constexpr (MASK) {
          const uint64_t keep = (i >> 3) ? keep1 : keep0;
          c.x &= (uint32_t)keep;
          c.y &= (uint32_t)(keep >> 32);
        }
        return as_bf16x8(fp8x8_to_bf16x8(c));
      } else {
        const uint8_t* va0 = vt + (i >> 3) * 32 * ROWB + voff[i & 7];
        return join_tr(lds_tr16(va0), lds_tr16(va0 + 16 * ROWB));
      }
    };
    u32x4 kf[8];
    if (active) {
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) kf[jj] = kread_h(0, jj);
    }
    const int nv1 = more ? issue_tile(kv0 + TT, buf ^ 1) : 0;
    if (active) {
      f32x4 s0[2][NQT], s1[2][NQT];
#pragma unroll
      for (int mm = 0; mm < 2; ++mm)
#pragma unroll
        for (int nt = 0; nt < NQT; ++nt) s0[mm][nt] = s1[mm][nt] = f32x4{0, 0, 0, 0};
#pragma unroll
      for (int jj = 0; jj < 8; ++jj)
#pragma unroll
        for (int nt = 0; nt < NQT; ++nt)
          s0[jj & 1][nt] = mfma16(as_bf16x8(kf[jj]), as_bf16x8(qv[nt][jj >> 1]), s0[jj & 1][nt]);
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) kf[jj] = kread_h(1, jj);
      const int lim0 = q0 + n + prefix;
      float a0[NQT], a1[NQT];
      bool g0, g1;
      bf16x8 pb0[NQT], pb1[NQT];
#pragma unroll
      for (int jj = 0; jj < 8; ++jj)
#pragma unroll
        for (int nt = 0; nt < NQT; ++nt)
          s1[jj & 1][nt] = mfma16(as_bf16x8(kf[jj]), as_bf16x8(qv[nt][jj >> 1]), s1[jj & 1][nt]);
      softmax_half<NQT, MASK, FP8>(s0, m, l, a0, g0, pb0, p.scale_log2, sm.u.pf.ks[buf], sm.u.pf.vs[buf], g, ntok,
                            0, kv0, lim0);
      if (g0) {
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
          for (int nt = 0; nt < NQT; ++nt) o[dt][nt] *= a0[nt];
      }
      bf16x8 vf[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) vf[i] = vread(i);
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int nt = 0; nt < NQT; ++nt) o[i][nt] = mfma16(vf[i], pb0[nt], o[i][nt]);
      softmax_half<NQT, MASK, FP8>(s1, m, l, a1, g1, pb1, p.scale_log2, sm.u.pf.ks[buf], sm.u.pf.vs[buf], g, ntok,
                            32, kv0, lim0);
      if (g1) {
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
          for (int nt = 0; nt < NQT; ++nt) o[dt][nt] *= a1[nt];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) vf[i] = vread(8 + i);
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int nt = 0; nt < NQT; ++nt) o[i][nt] = mfma16(vf[i], pb1[nt], o[i][nt]);
    }
    if (more) commit_tile(buf ^ 1, nv1, kv0 + TT);
  };
  // Tiles before the first one with a key past the valid rows or after the
  // block's first query position (bottom-right causal) need no mask.
  const int lim_first = min(kend - TT, q0 + prefix - (TT - 1));  // largest unmasked kv0
  const int n_int = lim_first < 0 ? 0 : lim_first / TT + 1;
  const int tfirst = kstart / TT;
  int kv0 = kstart, j = 0;
  // Interior tiles run in pairs, so each tile's LDS buffer is a constant and
  // its MFMA operand reads take lane offsets plus immediates (three 512-token
  // chunks after prefixes 0/2048/512, prefill-only: about 71 -> 68 us; 24
  // decode rows of 256-4096 tokens and two 512-token chunks: 68.2 -> 67.5 us).
  using F = std::integral_constant<bool, false>;
  using T = std::integral_constant<bool, true>;
  auto tiles = [&](auto codes_tag) {
    for (; kv0 + TT < kstop && tfirst + j + 1 < n_int; kv0 += 2 * TT, j += 2) {
      tile(F(), codes_tag, kv0, 0);
      tile(F(), codes_tag, kv0 + TT, 1);
    }
    for (; kv0 < kstop && tfirst + j < n_int; kv0 += TT, ++j) tile(F(), codes_tag, kv0, j);
    for (; kv0 < kstop; kv0 += TT, ++j) tile(T(), codes_tag, kv0, j);
  };
  // E4M3FN launches read every tile of a paged row as codes (the store of the
  // step's new tokens ran before the launch).
  if constexpr (FP8) {
    if (src_fp8) tiles(T());
    else tiles(F());
  } else {
    for (; kv0 + TT < kstop && tfirst + j + 1 < n_int; kv0 += 2 * TT, j += 2) {
      tile(F(), F(), kv0, 0);
      tile(F(), F(), kv0 + TT, 1);
    }
    for (; kv0 < kstop && tfirst + j < n_int; kv0 += TT, ++j) tile(F(), F(), kv0, j);
    for (; kv0 < kstop; kv0 += TT, ++j) tile(T(), F(), kv0, j);
  }

  if constexpr (SPLITK) {
    if (two) {
      // Record layout (floats, NQT * PF_REC_FLOATS per item): O as
      // [wave][nt][dt][lane] f32x4, then (m, l) as [wave][nt][lane] float2.
      constexpr int ML = 4 * NQT * 8 * 256;
      float* rec = p.partials + (size_t)item * (PF_REC_FLOATS * NQT);
      if (active) {
#pragma unroll
        for (int nt = 0; nt < NQT; ++nt) {
#pragma unroll
          for (int dt = 0; dt < 8; ++dt)
            store16_agent(rec + (((wave * NQT + nt) * 8 + dt) * 64 + lane) * 4,
                          __builtin_bit_cast(u32x4, o[dt][nt]));
          store8_agent(rec + ML + ((wave * NQT + nt) * 64 + lane) * 2,
                       u32x2{__float_as_uint(m[nt]), __float_as_uint(l[nt])});
        }
      }
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // records stored before the ticket
      __syncthreads();
      const int pair = p.hkv * p.HG;
      int* ticket = &p.counters[item - part * pair];
      if (tid == 0) {
        const uint32_t old = atomic_add_ret(ticket, 1u);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        sm.pf_ticket = (int)after_wait(old);
      }
      __syncthreads();
      if (sm.pf_ticket == 0) return;  // the partner item merges
      if (tid == 0) {
        atomicExch(ticket, 0);
        __hip_atomic_fetch_add(reinterpret_cast<uint32_t*>(p.ctrl) + EVENTS_OFFSET / 4 + EV_PF_SPLIT_MERGE, 1u,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      if (!active) return;
      const float* prec = p.partials + (size_t)(part ? item - pair : item + pair) * (PF_REC_FLOATS * NQT);
      // Merged in a fixed order (first half, then second), so the result's
      // rounding does not depend on which item arrived second.
      const float c = p.scale_log2;
#pragma unroll
      for (int nt = 0; nt < NQT; ++nt) {
        const float2 ml = load_partial2(prec + ML + ((wave * NQT + nt) * 64 + lane) * 2);
        const float m0 = part ? ml.x : m[nt], m1 = part ? m[nt] : ml.x;
        const float l0 = part ? ml.y : l[nt], l1 = part ? l[nt] : ml.y;
        const float mx = fmaxf(m0, m1);
        const float w0 = m0 == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(c * (m0 - mx));
        const float w1 = m1 == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(c * (m1 - mx));
        l[nt] = fmaf(l1, w1, l0 * w0);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const float* po = prec + (((wave * NQT + nt) * 8 + dt) * 64 + lane) * 4;
          const float2 a = load_partial2(po), b = load_partial2(po + 2);
          const f32x4 pv = f32x4{a.x, a.y, b.x, b.y};
          const f32x4 o0 = part ? pv : o[dt][nt], o1 = part ? o[dt][nt] : pv;
#pragma unroll
          for (int i = 0; i < 4; ++i) o[dt][nt][i] = fmaf(o1[i], w1, o0[i] * w0);
        }
      }
    }
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
// Launch shapes, one kernel instantiation each, so that every path is
// register-allocated without the code of paths the launch cannot take.
enum Mode : int {
  MODE_MIXED = 0,    // decode and prefill rows; prefill in 32-position blocks
  MODE_PREFILL = 1,  // prefill rows only; block size chosen per launch
  MODE_DECODE = 2,   // decode rows only
};

// FOLD: the launch carries the KV write of the step's new tokens (bf16
// pools): prefill tiles read new tokens from the new rows, and the tail tasks
// include the store.  A separate instantiation, so launches without it keep
// the prefill tile loop's smaller register footprint.
template <bool FP8, int MODE, bool FOLD = false>
__global__ void __launch_bounds__(NT, 2) paged_attention_kernel(Params p) {
  constexpr bool HAS_DEC = MODE != MODE_PREFILL;
  constexpr bool HAS_PF = MODE != MODE_DECODE;
  __shared__ Smem sm;
  __shared__ __attribute__((aligned(16))) uint8_t stage0[STAGE_BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t stage1[STAGE_BYTES];
  // decode: Q of the current and next item
  __shared__ __attribute__((aligned(16))) uint8_t qbuf[HAS_DEC ? 2 * QBUF : 16];
  // Prefill-only launches: the ranked units and the rows' geometry.
  constexpr bool PF_SORT = MODE == MODE_PREFILL;
  __shared__ uint32_t pf_units[PF_SORT ? PF_SORT_UNITS : 1];
  __shared__ int4 pf_geo[PF_SORT ? PF_SORT_ROWS : 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nrows = p.np + p.nd;

  const int per = (nrows + NT - 1) / NT;  // rows per thread, at most 4
  const int r0 = tid * per;
  // The host launches at least NLIST workgroups (lists without items cost a
  // workgroup nothing), so the list arithmetic is by a constant.
  constexpr int nlist = NLIST;
  const int list = blockIdx.x % nlist;


  // Prefill block size: a launch with decode rows uses 32 query positions
  // (the decode work hides the longest prefill item and 32 halves the key
  // tiles loaded per query); a prefill-only launch uses 16 when the heaviest
  // 32-position block would take more than twice a workgroup's fair share of
  // the work (the launch would wait on that one item) and not every such row
  // splits its keys (below), else 32.  Decode chunk:
  // d_chunk tokens (bf16 256, E4M3FN 512) when that still gives at least two
  // items per workgroup, else half of it (bf16 only: short launches need the
  // parallelism more than the longer items' lower per-token overhead).
  int bq = 32, dchunk = d_chunk<FP8>();
  // Item counts of this thread's rows under either choice (32-position
  // blocks / CHUNK, 16-position blocks / CHUNK_MIN), so the metadata is read
  // once.
  // cnt_d holds the second count minus the first, so choosing a count is an
  // addition: a choice between two array elements (alt ? cnt_b[i] : cnt_a[i])
  // was compiled into a load through a selected address, which kept both
  // arrays in scratch memory.
  int cnt_a[4], cnt_d[4], tmr[4];
  bool pf_long = false;  // prefill-only: a 32-position block spans over twice a workgroup's share
  {
    // tu: the longest block of this thread's rows that cannot split (a
    // short prefix, or at most 16 key tiles: pf_splits); a long row with more
    // than 16 tiles and a long prefix splits whenever it is long.
    int w = 0, tm = 0, dn = 0, tu = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = r0 + i;
      cnt_a[i] = cnt_d[i] = 0;
      tmr[i] = 0;
      if (i >= per || r >= nrows) continue;
      if (r < p.np) {
        int wr, tr;
        bool lp = false;
        pf_work(p, r, wr, tr, &lp);
        if (!lp || tr <= 16) tu = max(tu, tr);
        w += wr;
        tm = max(tm, tr);
        tmr[i] = tr;
        const int lq = p.cu_q[r + 1] - p.cu_q[r];
        cnt_a[i] = lq > 0 ? ((lq + 31) / 32) * p.hkv * p.HG : 0;
        cnt_d[i] = (lq > 0 ? ((lq + 15) / 16) * p.hkv * p.HG : 0) - cnt_a[i];
      } else {
        const int L = decode_len(p, r - p.np);
        dn += (L + d_chunk<FP8>() - 1) / d_chunk<FP8>();
        cnt_a[i] = max(1, (L + d_chunk<FP8>() - 1) / d_chunk<FP8>()) * p.hkv;
        cnt_d[i] = max(1, (L + d_chunk_min<FP8>() - 1) / d_chunk_min<FP8>()) * p.hkv - cnt_a[i];
      }
    }

#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      w += __shfl_xor(w, d, 64);
      tm = max(tm, __shfl_xor(tm, d, 64));
      dn += __shfl_xor(dn, d, 64);
      if constexpr (MODE == MODE_PREFILL && !FOLD) tu = max(tu, __shfl_xor(tu, d, 64));
    }
    if (lane == 0) {
      sm.wsum[wave] = w;
      sm.wmax[wave] = tm;
      sm.dsum[wave] = dn;
      sm.wumax[wave] = tu;
    }
    __syncthreads();
    int64_t wt = 0, dt = 0;
    int tmax = 0, tunsplit = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      wt += sm.wsum[i];
      tmax = max(tmax, sm.wmax[i]);
      dt += sm.dsum[i];
      tunsplit = max(tunsplit, sm.wumax[i]);
    }
    pf_long = MODE == MODE_PREFILL && (int64_t)tmax * gridDim.x > 2 * wt;
    if (pf_long) {
      // Rows that split their keys in two (below) halve their longest items
      // already, and take 32-position blocks, whose tiles cost half the LDS
      // operand reads per query (three 512-token chunks after prefixes
      // 0/2048/512: 65.7 -> 51.3 us; two after 0 and 1,024: 38.0 -> 37.8
      // us); the other rows take 16 only when a row this long cannot split
      // (tunsplit).  (A folded prefill-only instantiation would keep 16 for
      // all: its 32-position split items spilled registers; launch_attention
      // runs prefill-only launches without the KV write.)
      if (FOLD || (int64_t)tunsplit * gridDim.x > 2 * wt) bq = 16;
    }
    // (E4M3FN launches always take full 512-token items: measured 27.0 ->
    // 25.5 us on 16 rows of 64-1024 tokens and 54 -> 51 us on 24 rows of
    // 256-4096, where half items keep half the bytes in flight.)
    if (!FP8 && dt * p.hkv < 2 * (int64_t)gridDim.x) dchunk = d_chunk_min<FP8>();
    // E4M3FN mixed launches: a prefill row whose heaviest 32-position block
    // spans more key tiles than a workgroup's share of the launch (a decode
    // item counted as 4 tiles) uses 16-position blocks, which halves the
    // longest items; register-staged E4M3FN tiles make those items the
    // launch's critical path.  (With bf16 pools the extra tile reads cost
    // more than the shorter items gain.)
    if (tid == 0)
      sm.split_tiles = (FP8 && MODE == MODE_MIXED) ? (int)((4 * dt * p.hkv + wt) / gridDim.x) : (1 << 30);
    // Mixed launches: the share of workgroups that start with prefill items
    // follows the prefill share of the work (decode items counted as 4 tiles),
    // twice it, between a quarter and five eighths of the grid.  (Five eighths
    // measured best with a third of the work in prefill, a quarter with a
    // tenth.)
    if (tid == 0) {
      int permille = 500;
      if (MODE == MODE_MIXED) {
        const int64_t all = wt + 4 * dt * p.hkv;
        if (all > 0) permille = min(625, max(250, (int)(2000.0f * (float)wt / (float)all)));
      }
      sm.pf_first = (int)(gridDim.x * (uint32_t)permille / 1000u);
      // Long decode launches (six items or more per workgroup): each list
      // cycles through the kv heads instead of keeping one.  Whole lists
      // otherwise finished up to 15% apart (the same heads always on the
      // same lists); measured 146 -> 139 us on a 677 MB decode launch, while
      // short launches (about three items per workgroup) ran 3% slower
      // with it.
      sm.drot = dt * p.hkv >= 6 * (int64_t)gridDim.x;
      // Non-temporal K/V loads stream faster, but in mixed launches whose
      // prefill items are the critical path (decode work under 4 times the
      // prefill work) they made the launch slower: 24 decode rows of
      // 256-4096 tokens with two 512-token chunks 65.8 -> 66.5 us, while 64
      // rows of 512-4096 with one 1,024-token chunk went 146.4 -> 137.6 us.
      sm.kv_nt = MODE != MODE_MIXED || 4 * dt * p.hkv >= 4 * wt;
      sm.pf_split_thr = MODE == MODE_PREFILL ? (int)max((int64_t)16, 2 * wt / gridDim.x) : (1 << 30);
    }
    __syncthreads();
  }

  // Prefill-only launches: a row whose heaviest block spans more key tiles
  // than twice a workgroup's share of the work (and at least 16), after a
  // cached prefix at least as long as its chunk, is split in
  // two key ranges per item, merged by the range that finishes second, when
  // every item of the launch has a record slot (a ticket and pf_split_bytes
  // of records); such a row otherwise sets the launch's length alone.
  if constexpr (MODE == MODE_PREFILL) {
    int base_c = 0, extra_c = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (i >= per || r0 + i >= nrows) continue;
      // Split rows take 32-position blocks except in the folded instantiation.
      const bool sp = pf_splits(p, r0 + i, tmr[i], sm.pf_split_thr);
      const int c = cnt_a[i] + (bq == 16 && !(sp && !FOLD) ? cnt_d[i] : 0);
      base_c += c;
      if (sp) extra_c += c;
    }
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      base_c += __shfl_xor(base_c, d, 64);
      extra_c += __shfl_xor(extra_c, d, 64);
    }
    if (lane == 0) {
      sm.wsum[wave] = base_c;
      sm.dsum[wave] = extra_c;
    }
    __syncthreads();
    if (tid == 0) {
      const int all = sm.wsum[0] + sm.wsum[1] + sm.wsum[2] + sm.wsum[3];
      const int ext = sm.dsum[0] + sm.dsum[1] + sm.dsum[2] + sm.dsum[3];
      // Record slots of 32-position items (16 in the folded instantiation).
      const int cap = (int)(p.pf_split_bytes / (int64_t)(sizeof(float) * (size_t)PF_REC_FLOATS * (FOLD ? bq / 16 : 2)));
      if (ext == 0 || all + ext > cap || all + ext > MAX_COUNTERS) sm.pf_split_thr = 1 << 30;
    }
    __syncthreads();
    // No split after all: long rows take 16-position blocks.
    if (sm.pf_split_thr == (1 << 30) && pf_long) bq = 16;
  }

  // Per-row item counts -> exclusive prefix in sm.off (block-wide scan).
  int cnt[4];
  int local_sum = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool sp = MODE == MODE_PREFILL && r0 + i < p.np && pf_splits(p, r0 + i, tmr[i], sm.pf_split_thr);
    const bool alt = r0 + i < p.np ? ((bq == 16 && !(sp && !FOLD)) || tmr[i] > sm.split_tiles)
                                   : dchunk == d_chunk_min<FP8>();
    cnt[i] = cnt_a[i] + (alt ? cnt_d[i] : 0);
    if (sp) cnt[i] *= 2;
    local_sum += cnt[i];
  }
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
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (i < per && r0 + i < nrows) sm.off[r0 + i] = run;
    run += cnt[i];
  }
  if (tid == NT - 1) sm.off[nrows] = run;
  __syncthreads();
  const int total = sm.off[nrows];
  const int decode_base = sm.off[p.np];
  // Prefill-only launches: rank the units by their block's key count (ties:
  // lower row, then lower u, so the two halves of a split block stay adjacent
  // and item + hkv * HG is the second half of item).  Items are numbered in
  // that order instead of row by row, so every row's heaviest items start
  // first (four cold rows of 267-1,843 tokens: a later row's heaviest items
  // otherwise waited for the lighter items of the rows before it).
  const int per_unit = p.hkv * p.HG;
  bool sorted = false;
  if constexpr (PF_SORT) {
    // Launches that split rows keep the row order: there the first round of
    // workgroups pairs each CU's light item with a heavy half (two
    // 512-token chunks after prefixes 0 and 1,024: 37 us in row
    // order, 41 us ranked, where every CU started two heavy halves at once).
    const int units = decode_base / per_unit;
    sorted = p.np <= PF_SORT_ROWS && units <= PF_SORT_UNITS && (int64_t)units * p.np <= PF_SORT_COST &&
             sm.pf_split_thr == (1 << 30);
    if (sorted) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = r0 + i;
        if (i >= per || r >= p.np) continue;
        const PfRow g = pf_row(p, r);
        const int nqb = g.Lq > 0 ? (g.Lq + bq - 1) / bq : 0;
        const int mult = pf_splits(p, r, tmr[i], sm.pf_split_thr) ? 2 : 1;
        pf_geo[r] = int4{g.prefix, g.Lq, g.Lk, nqb | (mult << 16)};
      }
      __syncthreads();
      for (int r = 0; r < p.np; ++r) {
        const int4 g = pf_geo[r];
        const int nqb = g.w & 0xffff, mult = g.w >> 16;
        for (int u = tid; u < nqb * mult; u += NT) {
          const int b = nqb - 1 - u / mult;
          const int K = min(g.z, max(0, g.x + min(bq * (b + 1), g.y)));
          int rank = u - mult * pf_blocks_above(g, bq, K);
          for (int r2 = 0; r2 < p.np; ++r2) {
            const int4 g2 = pf_geo[r2];
            const int m2 = g2.w >> 16;
            const int above = pf_blocks_above(g2, bq, K);
            rank += m2 * above;
            if (r2 < r) rank += m2 * (pf_blocks_above(g2, bq, K - 1) - above);
          }
          pf_units[rank] = ((uint32_t)r << 16) | (uint32_t)u;
        }
      }
      __syncthreads();
    }
  }

  // Work lists.  Prefill items [0, decode_base) and decode items
  // [decode_base, total) form two families; item i of a family belongs to list
  // i % nlist of that family (E4M3FN decode items: by groups of hkv, see
  // dec_index) and workgroup b serves list b % nlist of both, so
  // the lists' fetch counters are separate addresses (and, with round-robin
  // dispatch and 8 kv heads, one kv head's prefill tiles stay on one XCD's
  // L2).  Workgroups of a list start with different families and take the
  // other one when theirs is exhausted, so MFMA-bound prefill items
  // and HBM-bound decode items run side by side from the start.  A list's
  // counter is zero when a launch starts.  Every workgroup stops after its
  // first fetch past the list, so a launch makes exactly count + workgroups
  // fetches on a list (fewer by the static first items below), and the
  // workgroup that makes the last one (the one returning the largest value)
  // resets the counter: every other workgroup has made its last fetch by
  // then.  Fetches that add 0 (decode loop padding) may follow the reset;
  // their results are ignored.  No counter is contended by a completion count.
  const uint32_t wgs = (uint32_t)((gridDim.x - list + nlist - 1) / nlist);
  // Family taken first (0 prefill, 1 decode): workgroups below pf_first (a
  // quarter to five eighths of the grid) start with prefill, the rest with
  // decode.
  // The dispatcher fills every CU's first workgroup slot before any second
  // one, so with a half the workgroups b and b + grid/2 share a CU and each CU
  // pairs an MFMA-bound prefill workgroup with an HBM-bound decode one.
  const int pf_first = sm.pf_first;  // workgroups that start with the prefill family
  const int first = (int)blockIdx.x >= pf_first ? 1 : 0;
  // Static first items: the workgroups of a list that start with a family
  // (all of them when the list has items in one family only) take that
  // family's first items by their index, without a fetch; fetched relative
  // indices start after them (fetch value f is relative index S + f), and a
  // family is fetched count - S + wgs times per launch (one out-of-list fetch
  // per workgroup).
  const int member = blockIdx.x / nlist;  // index of this workgroup in its list
  const int wfirst0 = pf_first > list ? (pf_first - list + nlist - 1) / nlist : 0;  // prefill-first members
  uint32_t fcount[2];
#pragma unroll
  for (int fam = 0; fam < 2; ++fam) {
    const int fsize = fam ? total - decode_base : decode_base;
    fcount[fam] = fam ? (uint32_t)dec_count(list, nlist, FP8 ? p.hkv : 1, fsize)
                      : (list < fsize ? (uint32_t)((fsize - list + nlist - 1) / nlist) : 0u);
  }
  const bool both = fcount[0] > 0 && fcount[1] > 0;
  if (tid == 0) sm.salt = 0;
  for (int pass = 0; pass < 2; ++pass) {
    const int fam = first ^ pass;
    const int fbase = fam ? decode_base : 0;
    const uint32_t count = fcount[fam];
    // A list without items this launch is not touched: its counter stays zero.
    if (count == 0) continue;
    const int wfam = both ? (fam ? (int)wgs - wfirst0 : wfirst0) : (int)wgs;  // members starting here
    const int jfam = both ? (fam ? member - wfirst0 : member) : member;      // this one's index among them
    const bool starts_here = !both || fam == first;
    const uint32_t S = min(count, (uint32_t)wfam);  // static items of this family
    const bool has_static = starts_here && jfam >= 0 && (uint32_t)jfam < count;
    uint32_t* ctr = reinterpret_cast<uint32_t*>(p.ctrl) + (fam * NLIST + list) * CTRL_STRIDE;
    const uint32_t base = 0u - S;  // fetch value of relative index 0: relative = fetch value + S
    if (tid == 0) sm.item = has_static ? (uint32_t)jfam : atomicAdd(ctr, 1u) - base;  // relative index
    __syncthreads();

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
      const int item =
          fam ? fbase + dec_index(list, nlist, FP8 ? p.hkv : 1, (int)rel) : fbase + list + (int)rel * nlist;
      if (PF_SORT && sorted && !fam) return (int)(pf_units[item / per_unit] >> 16);
      for (int r = tid; r < nrows; r += NT)
        if (sm.off[r] <= item && item < sm.off[r + 1]) sm.row = r;
      __syncthreads();
      return sm.row;
    };

    uint32_t rel = sm.item;
    __syncthreads();
    int r = resolve(rel);
    while (r >= 0) {
      // sm.salt is always 0; reading it here keeps the lane-derived values of
      // the two item paths from being hoisted out of the loop, where they
      // would all stay live at once.
      const int ltid = tid + sm.salt;
      if (HAS_PF && r < p.np) {
        const int item = list + (int)rel * nlist;
        if constexpr (MODE == MODE_PREFILL) {
          bool sp = false;
          {
            int wr = 0, tr = 0;
            pf_work(p, r, wr, tr);
            sp = pf_splits(p, r, tr, sm.pf_split_thr);
          }
          // Split items only where the row splits (32-position blocks, 16 in
          // the folded instantiation); other items keep the tile loop
          // compiled without the split's range and merge code.
          const int lr = sorted ? (int)(pf_units[item / per_unit] & 0xffffu) * per_unit + item % per_unit
                                : item - sm.off[r];
          if (sp) {
            if constexpr (!FOLD) prefill_item<FP8, 2, FOLD, true>(p, sm, stage0, stage1, r, lr, ltid, item, true);
            else prefill_item<FP8, 1, FOLD, true>(p, sm, stage0, stage1, r, lr, ltid, item, true);
          }
          else if (bq == 16) prefill_item<FP8, 1, FOLD>(p, sm, stage0, stage1, r, lr, ltid);
          else prefill_item<FP8, 2, FOLD>(p, sm, stage0, stage1, r, lr, ltid);
        } else if constexpr (HAS_PF) {
          // The row's items are 16-position blocks exactly when the item
          // counts above took them so (tmr > split_tiles, E4M3FN launches).
          const int lr = item - sm.off[r];
          int wr = 0, tr = 0;
          if constexpr (FP8) pf_work(p, r, wr, tr);
          if (FP8 && tr > sm.split_tiles) prefill_item<FP8, FP8 ? 1 : 2, FOLD>(p, sm, stage0, stage1, r, lr, ltid);
          else prefill_item<FP8, 2, FOLD>(p, sm, stage0, stage1, r, lr, ltid);
        }
        // The next item is fetched only now: fetching ahead would let a
        // workgroup claim a second item before a late-starting one takes its
        // first.
        uint32_t next = 0;
        if (tid == 0) next = atomicAdd(ctr, 1u) - base;
        rel = advance(next);
        r = resolve(rel);
        continue;
      }
      // The rest of this decode list is one streaming decode run.
      if constexpr (HAS_DEC) {
        if (MODE == MODE_DECODE || sm.kv_nt)
          decode_run<FP8, FOLD, true>(p, sm, stage0, stage1, qbuf, list, nlist, count, base, ctr, decode_base, nrows,
                                      rel, r, dchunk, ltid);
        else
          decode_run<FP8, FOLD, false>(p, sm, stage0, stage1, qbuf, list, nlist, count, base, ctr, decode_base, nrows,
                                       rel, r, dchunk, ltid);
      }
      break;
    }
    if (tid == 0 && sm.item == count + wgs - 1u) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
  }
  tail_tasks<FP8, FOLD>(p, sm, list, nlist, decode_base, dchunk, tid);

  // Rows that belong to no decode or prefill row (the capacity padding of a
  // captured step) get zeros, so every output row is defined.
  const int64_t covered = (int64_t)p.q_off_prefill + (p.np_all > 0 ? max(p.cu_q_all[p.np_all], 0) : 0);
  if (covered < p.num_q_rows) {
    const int per_row = p.hkv * p.G * HD / 8;  // 16-byte pieces per output row
    const int64_t pieces = (p.num_q_rows - covered) * per_row;
    for (int64_t i = (int64_t)blockIdx.x * NT + tid; i < pieces; i += (int64_t)gridDim.x * NT) {
      const int64_t row = covered + i / per_row;
      *reinterpret_cast<u32x4*>(p.out + row * p.out_stride + 8 * (i % per_row)) = u32x4{0, 0, 0, 0};
    }
  }
}

using AttnKernel = void (*)(Params);

// The instantiations, indexed [fold][fp8][mode].
AttnKernel attn_kernel(bool fold, bool fp8, int mode) {
  static const AttnKernel table[2][2][3] = {
      {{paged_attention_kernel<false, MODE_MIXED>, paged_attention_kernel<false, MODE_PREFILL>,
        paged_attention_kernel<false, MODE_DECODE>},
       {paged_attention_kernel<true, MODE_MIXED>, paged_attention_kernel<true, MODE_PREFILL>,
        paged_attention_kernel<true, MODE_DECODE>}},
      // Prefill-only launches and E4M3FN launches with prefill rows never
      // carry the KV write (launch_attention runs the store kernel first).
      {{paged_attention_kernel<false, MODE_MIXED, true>, nullptr, paged_attention_kernel<false, MODE_DECODE, true>},
       {nullptr, nullptr, paged_attention_kernel<true, MODE_DECODE, true>}},
  };
  return table[fold ? 1 : 0][fp8 ? 1 : 0][mode];
}

using DirectKernel = void (*)(Params, int, int, int);
DirectKernel direct_kernel(bool fold, bool fp8) {
  static const DirectKernel table[2][2] = {{decode_direct_kernel<false, false>, decode_direct_kernel<true, false>},
                                           {decode_direct_kernel<false, true>, decode_direct_kernel<true, true>}};
  return table[fold ? 1 : 0][fp8 ? 1 : 0];
}
// Decode-only launches whose direct grid of the longest chunks (one workgroup
// per chunk the tables can hold) is at most this many times what the GPU
// holds at once run the direct kernel (bf16, E4M3FN pools); longer launches
// run the work lists.  Measured on rows of 64-8192 tokens: the direct kernel
// wins up to these sizes (16 rows of 64-1024 tokens 30 -> 15 us, 24 rows of
// 256-4096 53 -> 51 us bf16 and 41 -> 37 us E4M3FN), the work lists beyond.
constexpr int DIRECT_MAX_ROUNDS[2] = {4, 2};
constexpr int DIRECT_CHUNK_MAX = 1024;  // tokens

// Compute units and, per instantiation, the workgroups one CU holds at once
// (registers and LDS of that kernel), cached per device.  A persistent launch
// of CUs x that many workgroups keeps every workgroup resident.
struct DeviceShape {
  int cus = 0;
  int wallclock_khz = 0;  // s_memrealtime rate
  int wg_per_cu[2][2][3] = {};
  int wg_direct[2] = {};  // decode_direct_kernel (without the KV write), by pool format
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
    if (hipDeviceGetAttribute(&s.cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipDeviceGetAttribute(&s.wallclock_khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess)
      return fail(SLO_ERR_HIP, "hipDeviceGetAttribute failed");
    if (s.wallclock_khz <= 0) s.wallclock_khz = 100000;
    for (int fold = 0; fold < 2; ++fold)
      for (int fp8 = 0; fp8 < 2; ++fp8)
        for (int mode = 0; mode < 3; ++mode) {
          const AttnKernel k = attn_kernel(fold, fp8, mode);
          if (!k) continue;
          int n = 0;
          if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, NT, 0) != hipSuccess)
            return fail(SLO_ERR_HIP, "occupancy query failed");
          s.wg_per_cu[fold][fp8][mode] = std::max(1, n);
        }
    for (int fp8 = 0; fp8 < 2; ++fp8) {
      int n = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, direct_kernel(false, fp8), NT, 0) != hipSuccess)
        return fail(SLO_ERR_HIP, "occupancy query failed");
      s.wg_direct[fp8] = std::max(1, n);
    }
    cache[dev] = s;
    ready[dev] = true;
  }
  *out = cache[dev];
  return SLO_OK;
}

size_t partial_floats(int64_t items, int G) { return (size_t)items * G * PREC; }

}  // namespace slo

using namespace slo;

extern "C" int slo_attention_workspace_bytes(int32_t max_decode_rows, int32_t max_decode_len, int32_t num_heads,
                                             int32_t num_kv_heads, int32_t head_dim, size_t* bytes) {
  if (!bytes || max_decode_rows < 0 || max_decode_len < 0 || num_kv_heads <= 0 || num_heads <= 0 ||
      num_heads % num_kv_heads)
    return fail(SLO_ERR_INVALID, "workspace_bytes: bad arguments");
  if (head_dim != HD) return fail(SLO_ERR_UNSUPPORTED, "workspace_bytes: head_dim must be 128");
  const int64_t chunks = (max_decode_len + CHUNK_MIN - 1) / CHUNK_MIN;
  const int64_t items = (int64_t)max_decode_rows * std::max<int64_t>(1, chunks) * num_kv_heads;
  *bytes = PARTIALS_OFFSET + sizeof(float) * partial_floats(items, num_heads / num_kv_heads) + PF_SPLIT_BYTES;
  return SLO_OK;
}

namespace slo {

// One launch with workspace `ws` of `ws_bytes` bytes.  `sized` is true for a
// caller-sized workspace (slo_paged_attention: at least
// slo_attention_workspace_bytes), false for the library's static scratch,
// which must hold this launch's decode partials, or split prefill records of
// up to PF_SPLIT_BYTES, after the control area.
int launch_attention(const slo_paged_attention_args* a, void* ws, size_t ws_bytes, bool sized, slo_stream_t stream) {
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
  if (!a->q || !a->out || !ws) return fail(SLO_ERR_INVALID, "paged_attention: null q/out/workspace");
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
          a->v_row_stride >= (1 << 25) || a->k_row_stride < (int64_t)a->num_kv_heads * HD ||
          a->v_row_stride < (int64_t)a->num_kv_heads * HD ||
          (reinterpret_cast<uintptr_t>(a->k) % 16) || (reinterpret_cast<uintptr_t>(a->v) % 16))
        return fail(SLO_ERR_INVALID,
                    "paged_attention: contiguous K/V must be 16-byte aligned bf16 rows of at least num_kv_heads * 128");
    }
  }
  const bool store = a->store_slot_mapping != nullptr;
  // The KV write runs inside launches with decode rows except on E4M3FN
  // pools with prefill rows; elsewhere it runs as the store kernel first and
  // the launch reads the pool (same bytes and outputs).  The folded E4M3FN
  // instantiations with prefill rows spilled registers and measured slower
  // (108 against 72 us on 24 decode rows of 256-4096 tokens beside two
  // 512-token chunks); prefill-only launches without the write split their
  // long rows' keys over 32-position blocks, which the folded instantiation
  // cannot (three 512-token chunks after prefixes 0/2048/512: 74.7 -> 55.1 us
  // for the step; four cold rows of 267-1,843 tokens 91.1 -> 90.1 us), while
  // the mixed launch gains from the fold (65.5 against 70.6 us).
  const bool fold = store && do_dec && !(fp8 && do_pf);
  if (store) {
    if (fp8 && !(a->store_scale_floor > 0.0f))
      return fail(SLO_ERR_INVALID, "paged_attention: the E4M3FN KV write needs store_scale_floor > 0");
    if (fp8 && a->num_heads > 8 * a->num_kv_heads)
      return fail(SLO_ERR_UNSUPPORTED, "paged_attention: the E4M3FN KV write in the launch needs <= 8 query heads per kv head");
    if (!a->k_cache || !a->v_cache || a->num_blocks <= 0 || a->block_size <= 0)
      return fail(SLO_ERR_INVALID, "paged_attention: the KV write needs the pool");
    const int64_t row = (int64_t)a->num_kv_heads * HD;
    if (!a->new_k || !a->new_v || a->num_new_rows != a->num_q_rows || a->new_k_row_stride != row ||
        a->new_v_row_stride != row || (reinterpret_cast<uintptr_t>(a->new_k) % 16) ||
        (reinterpret_cast<uintptr_t>(a->new_v) % 16))
      return fail(SLO_ERR_INVALID,
                  "paged_attention: new K/V must be contiguous 16-byte aligned bf16 rows, one per query row");
  }
  if (store && !fold) {
    const int rc = slo_store_kvcache(a->new_k, a->new_k_row_stride, a->new_v, a->new_v_row_stride,
                                     a->store_slot_mapping, a->num_new_rows, a->num_kv_heads, HD, a->kv_dtype,
                                     const_cast<void*>(a->k_cache), const_cast<void*>(a->v_cache),
                                     const_cast<float*>(a->k_scale), const_cast<float*>(a->v_scale),
                                     (int64_t)a->num_blocks * a->block_size, a->store_scale_floor, stream);
    if (rc) return rc;
  }
  // Workspace: control words, split-K tickets, then decode partials (or, in
  // prefill-only launches, split prefill records).
  const int dec_len_cap = do_dec ? a->decode_table_width * a->block_size : 0;
  int64_t pf_split_bytes = PF_SPLIT_BYTES;
  if (sized) {
    size_t need = 0;
    int rc = slo_attention_workspace_bytes(do_dec ? a->num_decode : 0, dec_len_cap, a->num_heads, a->num_kv_heads, HD,
                                           &need);
    if (rc) return rc;
    if (ws_bytes < need) return fail(SLO_ERR_WORKSPACE, "paged_attention: workspace too small");
  } else {
    const int64_t chunks = (dec_len_cap + CHUNK_MIN - 1) / CHUNK_MIN;
    const size_t dec_bytes =
        do_dec ? sizeof(float) * partial_floats((int64_t)a->num_decode * std::max<int64_t>(1, chunks) * a->num_kv_heads, G)
               : 0;
    if (ws_bytes < PARTIALS_OFFSET || dec_bytes > ws_bytes - PARTIALS_OFFSET) {
      char msg[200];
      snprintf(msg, sizeof msg,
               "paged_attention_noalloc: %d decode rows of up to %d tokens need %zu bytes of split-K partials; the "
               "static scratch holds %zu",
               a->num_decode, dec_len_cap, dec_bytes, ws_bytes - PARTIALS_OFFSET);
      return fail(SLO_ERR_UNSUPPORTED, msg);
    }
    pf_split_bytes = std::min<int64_t>(PF_SPLIT_BYTES, (int64_t)(ws_bytes - PARTIALS_OFFSET));
  }
  if (reinterpret_cast<uintptr_t>(ws) % 256) return fail(SLO_ERR_INVALID, "paged_attention: workspace must be 256-byte aligned");

  DeviceShape ds;
  const int rc = device_shape(&ds);
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
  char* wsb = static_cast<char*>(ws);
  p.ctrl = reinterpret_cast<int*>(wsb);
  p.counters = reinterpret_cast<int*>(wsb + CTRL_BYTES);
  p.partials = reinterpret_cast<float*>(wsb + PARTIALS_OFFSET);
  p.pf_split_bytes = pf_split_bytes;
  p.sslots = fold ? a->store_slot_mapping : nullptr;
  p.nk = static_cast<const uint16_t*>(a->new_k);
  p.nv = static_cast<const uint16_t*>(a->new_v);
  p.nk_stride = a->new_k_row_stride;
  p.nv_stride = a->new_v_row_stride;
  p.nnew = fold ? a->num_new_rows : 0;
  p.scale_floor = a->store_scale_floor;
  p.num_slots = (int64_t)a->num_blocks * a->block_size;
  // A merge task waits up to 200 ms for its chunks (a whole decode launch
  // takes well under a millisecond) before it gives up and reports it.
  // SLO_ATTN_MERGE_WAIT_US overrides the bound (0 makes every merge whose
  // chunks are not all in give up, which the tests use to run that path).
  int64_t wait_us = 200000;
  if (const char* e = std::getenv("SLO_ATTN_MERGE_WAIT_US")) wait_us = std::max(0LL, std::atoll(e));
  p.merge_wait_ticks = wait_us * ds.wallclock_khz / 1000;
  p.cu_q_all = a->num_prefill > 0 ? a->prefill_cu_q : nullptr;
  p.np_all = a->num_prefill > 0 && a->prefill_cu_q ? a->num_prefill : 0;

  // Upper bound on the item count from host-known shapes only.
  int64_t bound = 0;
  if (do_dec) bound += (int64_t)p.nd * ((dec_len_cap + CHUNK_MIN - 1) / CHUNK_MIN) * p.hkv;
  if (do_pf) {
    const int64_t tq = std::max<int64_t>(0, a->num_q_rows - a->num_decode);
    bound += (tq / BQ_MIN + p.np) * p.hkv * p.HG;
  }
  // The E4M3FN instantiation only where the launch reads the pool: a launch of
  // cold prefill rows (new K/V only) runs the bf16 one, which holds fewer
  // registers.
  const bool fp8_reads = fp8 && (do_dec || (do_pf && p.ptab != nullptr));
  const int mode = do_dec && do_pf ? MODE_MIXED : do_pf ? MODE_PREFILL : MODE_DECODE;
  // With the KV write folded in, the pool's format decides the instantiation
  // (its store quantises); otherwise what the launch reads does.
  const bool kfp8 = fold ? fp8 : fp8_reads;
  const AttnKernel kernel = attn_kernel(fold, kfp8, mode);
  const int64_t slots = (int64_t)ds.cus * ds.wg_per_cu[fold ? 1 : 0][kfp8 ? 1 : 0][mode];
  if (mode == MODE_DECODE) {
    // The shortest chunks whose grid (one workgroup per chunk the tables can
    // hold) is at most 1.5 times what the GPU holds at once: rows shorter
    // than the tables' width leave part of the grid without tokens, so a grid
    // a little above the GPU still runs in one round.  Else the longest, when
    // their grid fits DIRECT_MAX_ROUNDS times.  (With a bound of 1x, 24 rows
    // of 256-4096 tokens at 16/4 heads took 1,024-token chunks and left half
    // the GPU idle: 36.2 us bf16 and 23.0 us E4M3FN, against 28.9 and 19.3
    // with the 512-token chunks the 1.5x bound picks; at 32/8 heads and on 16
    // rows of 64-1,024 tokens the choice does not change.)
    const int64_t held = (int64_t)ds.cus * ds.wg_direct[kfp8 ? 1 : 0];
    const int step_tokens = kfp8 ? d_step<true>() : d_step<false>();
    const int max_steps = DIRECT_CHUNK_MAX / step_tokens;
    for (int steps = 2; steps <= max_steps; steps *= 2) {
      const int ch = steps * step_tokens;
      const int nch_cap = std::max(1, (dec_len_cap + ch - 1) / ch);
      const int64_t dgrid = ((int64_t)p.nd * nch_cap + 7) / 8 * 8 * p.hkv;
      if (dgrid > (steps == max_steps ? DIRECT_MAX_ROUNDS[kfp8 ? 1 : 0] * held : held + held / 2)) continue;
      int spread = !kfp8 && p.hkv % 8 == 0 && dgrid <= 2 * held ? 1 : 0;
      void* dargs[] = {&p, const_cast<int*>(&nch_cap), &steps, &spread};
      if (hipLaunchKernel(reinterpret_cast<const void*>(direct_kernel(fold, kfp8)), dim3((unsigned)dgrid), dim3(NT),
                          dargs, 0, static_cast<hipStream_t>(stream)) != hipSuccess)
        return fail(SLO_ERR_HIP, "paged_attention: launch failed");
      return check_launch("paged_attention");
    }
  }
  // At least one workgroup per work list (the kernel's list arithmetic
  // assumes NLIST lists).
  const int grid = (int)std::max<int64_t>(NLIST, std::min<int64_t>(bound, slots));
  void* kargs[] = {&p};
  if (hipLaunchKernel(reinterpret_cast<const void*>(kernel), dim3(grid), dim3(NT), kargs, 0,
                      static_cast<hipStream_t>(stream)) != hipSuccess)
    return fail(SLO_ERR_HIP, "paged_attention: launch failed");
  return check_launch("paged_attention");
}

// The allocation-free entry's workspace: one array per GPU, zero when the
// code object is loaded, its control words and tickets zero again after every
// launch.  In host code `scratch` is only a stand-in for the device symbol:
// kernels get the address hipGetSymbolAddress returns for the current device.
constexpr size_t SCRATCH_BYTES = 64u << 20;
static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

int scratch_address(void** out) {
  static std::mutex mu;
  static void* addr[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return fail(SLO_ERR_HIP, "hipGetDevice failed");
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr)
      return fail(SLO_ERR_HIP, "paged_attention_noalloc: hipGetSymbolAddress of the static scratch failed");
    addr[dev] = ptr;
  }
  *out = addr[dev];
  return SLO_OK;
}

}  // namespace slo

extern "C" int slo_paged_attention(const slo_paged_attention_args* a, slo_stream_t stream) {
  if (!a) return fail(SLO_ERR_INVALID, "paged_attention: null args");
  return launch_attention(a, a->workspace, a->workspace_bytes, true, stream);
}

extern "C" int slo_paged_attention_noalloc(const slo_paged_attention_args* a, slo_stream_t stream) {
  if (!a) return fail(SLO_ERR_INVALID, "paged_attention_noalloc: null args");
  if (a->workspace || a->workspace_bytes)
    return fail(SLO_ERR_INVALID, "paged_attention_noalloc: workspace must be NULL (the static scratch is used)");
  const bool any = ((a->phases & SLO_PHASE_DECODE) && a->num_decode > 0) ||
                   ((a->phases & SLO_PHASE_PREFILL) && a->num_prefill > 0);
  void* ws = nullptr;
  if (any) {
    const int rc = scratch_address(&ws);
    if (rc) return rc;
  }
  return launch_attention(a, ws, SCRATCH_BYTES, false, stream);
}

extern "C" int slo_attention_workspace_check(const void* workspace, size_t workspace_bytes, uint32_t* events,
                                             slo_stream_t stream) {
  if (!workspace && !workspace_bytes) {  // the static scratch of slo_paged_attention_noalloc on this device
    void* ws = nullptr;
    const int rc = scratch_address(&ws);
    if (rc) return rc;
    workspace = ws;
    workspace_bytes = SCRATCH_BYTES;
  }
  if (!workspace || workspace_bytes < PARTIALS_OFFSET)
    return fail(SLO_ERR_INVALID, "workspace_check: workspace missing or smaller than its control area");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cap) != hipSuccess) return fail(SLO_ERR_HIP, "workspace_check: hipStreamIsCapturing failed");
  if (cap != hipStreamCaptureStatusNone) return fail(SLO_ERR_INVALID, "workspace_check: the stream is being captured");
  if (hipStreamSynchronize(s) != hipSuccess) return fail(SLO_ERR_HIP, "workspace_check: hipStreamSynchronize failed");
  std::vector<uint32_t> words(PARTIALS_OFFSET / 4);
  if (hipMemcpy(words.data(), workspace, PARTIALS_OFFSET, hipMemcpyDeviceToHost) != hipSuccess)
    return fail(SLO_ERR_HIP, "workspace_check: hipMemcpy failed");
  // Event counters: handed out, then cleared, so each event is reported once.
  uint32_t ev[EV_COUNT];
  std::memcpy(ev, words.data() + EVENTS_OFFSET / 4, sizeof ev);
  if (events) std::memcpy(events, ev, sizeof ev);
  bool any = false;
  for (int i = 0; i < EV_COUNT; ++i) any = any || ev[i];
  if (any) {
    const uint32_t zeros[EV_COUNT] = {};
    if (hipMemcpy(static_cast<char*>(const_cast<void*>(workspace)) + EVENTS_OFFSET, zeros, sizeof zeros,
                  hipMemcpyHostToDevice) != hipSuccess)
      return fail(SLO_ERR_HIP, "workspace_check: hipMemcpy failed");
  }
  static const char* const family[3] = {"prefill item", "decode item", "tail task"};
  for (size_t i = 0; i < words.size(); ++i) {
    if (i * 4 >= (size_t)TRASH_OFFSET && i * 4 < (size_t)CTRL_BYTES) continue;  // trash and event lines
    if (!words[i]) continue;
    char msg[160];
    if (i * 4 < (size_t)TRASH_OFFSET) {
      const int line = (int)(i / CTRL_STRIDE);
      snprintf(msg, sizeof msg, "workspace_check: %s counter of list %d (word %d) is %u, not 0",
               family[line / NLIST], line % NLIST, (int)(i % CTRL_STRIDE), words[i]);
    } else {
      snprintf(msg, sizeof msg, "workspace_check: ticket %zu is %#x, not 0", i - CTRL_BYTES / 4, words[i]);
    }
    return fail(SLO_ERR_STATE, msg);
  }
  if (ev[EV_MERGE_GAVE_UP]) {
    char msg[200];
    snprintf(msg, sizeof msg,
             "workspace_check: %u split-K merges gave up waiting for their chunks since the last check; those "
             "decode outputs were not written (workgroups of the launch could not run in time)",
             ev[EV_MERGE_GAVE_UP]);
    return fail(SLO_ERR_STATE, msg);
  }
  return SLO_OK;
}
