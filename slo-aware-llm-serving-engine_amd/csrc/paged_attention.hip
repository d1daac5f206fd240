// Ragged mixed prefill/decode paged attention for gfx950 (MI355X), one launch.
//
// Replaces the per-phase flash-attn calls of forward_mixed
// (nanovllm/layers/mixed_attention.py:36-57) and of the V0 branches of
// Attention.forward (nanovllm/layers/attention.py:68-78).
//
// Work list.  Every workgroup (4 wavefronts) first derives, from the metadata
// alone, the number of work items of every row and their exclusive prefix
// (prefill rows first, then decode rows), then pulls item indices from a
// device counter until the list is exhausted.  The grid is sized from
// capacities, never from device data, so the launch can be recorded in a HIP
// graph.  The counter and the split-K tickets reset themselves at the end of
// every launch, so no memset is ever needed.
//
//  * Prefill item (row r, query block of BQ positions, kv head h): each
//    wavefront owns one of the G query heads that share kv head h, for the
//    same BQ positions, so the K/V tiles staged in LDS serve all G heads.  The
//    contraction runs on bf16 MFMA (v_mfma_f32_16x16x32_bf16) in the
//    transposed form S^T = K Q^T, O^T += V^T P^T, which keeps each query
//    column's softmax statistics lane-local: the S^T accumulator is the B
//    operand of the PV product without any data movement, and V^T comes from
//    the natural [token][d] LDS tile through ds_read_b64_tr_b16.
//  * Decode item (row b, chunk of 256 tokens, kv head h): each wavefront takes
//    64 tokens; the G query heads sharing h are the MFMA columns, K goes from
//    HBM straight into MFMA A-operand registers, V is staged in LDS for the
//    transposed read.  The 4 wavefronts merge in LDS; when a row has several
//    chunks, each writes an (m, l, acc) partial and the last chunk to finish
//    (device-scope ticket) merges them (docs/project_manual.md:643-650).
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

constexpr int HD = 128;         // head_dim this kernel implements
constexpr int NT = 256;         // threads per workgroup (4 wavefronts)
constexpr int TT = 64;          // tokens per wavefront tile
constexpr int CHUNK = 4 * TT;   // decode split-K chunk
constexpr int ROW = HD + 8;     // LDS row pitch in bf16 (272 bytes)
constexpr int MAX_ROWS = 2048;  // decode + prefill rows per launch
constexpr int MAX_G = 16;       // query heads per kv head
constexpr int CTRL_BYTES = 256;
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
  int32_t nd;  // decode rows taking part in this launch
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
  int* ctrl;      // [0] next item, [1] finished workgroups
  int* counters;  // split-K tickets, [num_decode * hkv]
  float* partials;
};

template <int NQT>
struct Smem {
  union {
    uint16_t dec_v[4][TT * ROW];  // decode: one V tile per wavefront
    struct {
      uint16_t k[TT * ROW];
      uint16_t v[TT * ROW];
      float ks[TT];
      float vs[TT];
    } pf;
    struct {
      float o[4][MAX_G][HD];
      float m[4][MAX_G];
      float l[4][MAX_G];
    } mg;
  } u;
  int off[MAX_ROWS + 1];
  int wsum[4];
  int item;
  int row;
  int last;
};

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ u32x2 ld8(const void* p) { return *reinterpret_cast<const u32x2*>(p); }
__device__ __forceinline__ void st16(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }

__device__ __forceinline__ u32x4 fp8x8_to_bf16x8(const u32x2& w) {
  const u32x2 a = fp8x4_to_bf16x4(w.x), b = fp8x4_to_bf16x4(w.y);
  u32x4 r;
  r.x = a.x;
  r.y = a.y;
  r.z = b.x;
  r.w = b.y;
  return r;
}

__device__ __forceinline__ s16x4 lds_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(const_cast<uint16_t*>(p)));
}

__device__ __forceinline__ bf16x8 join_tr(const s16x4& a, const s16x4& b) {
  u32x4 r;
  r.x = (uint32_t)(uint16_t)a[0] | ((uint32_t)(uint16_t)a[1] << 16);
  r.y = (uint32_t)(uint16_t)a[2] | ((uint32_t)(uint16_t)a[3] << 16);
  r.z = (uint32_t)(uint16_t)b[0] | ((uint32_t)(uint16_t)b[1] << 16);
  r.w = (uint32_t)(uint16_t)b[2] | ((uint32_t)(uint16_t)b[3] << 16);
  return as_bf16x8(r);
}

__device__ __forceinline__ int decode_len(const Params& p, int b) {
  const int L = p.dlens[b];
  return min(max(L, 0), p.dtab_width * p.block_size);
}

template <int NQT>
__device__ __forceinline__ int row_items(const Params& p, int r) {
  constexpr int BQ = 16 * NQT;
  if (r < p.np) {
    const int lq = p.cu_q[r + 1] - p.cu_q[r];
    return lq > 0 ? ((lq + BQ - 1) / BQ) * p.hkv * p.HG : 0;
  }
  const int L = decode_len(p, r - p.np);
  return max(1, (L + CHUNK - 1) / CHUNK) * p.hkv;
}

// ---------------------------------------------------------------- decode item
template <bool FP8, int NQT>
__device__ void decode_item(const Params& p, Smem<NQT>& sm, int b, int local, int dindex) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int G = p.G;
  const int h = local % p.hkv, c = local / p.hkv;
  const int L = decode_len(p, b);
  const int nch = max(1, (L + CHUNK - 1) / CHUNK);
  const int t0 = c * CHUNK + wave * TT;
  int ntok = min(max(L - t0, 0), TT);
  int64_t slot0 = 0;
  if (ntok > 0) {
    const int page = p.dtab[(int64_t)b * p.dtab_stride + t0 / p.block_size];
    if (page < 0 || page >= p.num_blocks) ntok = 0;  // never dereference padding
    else slot0 = (int64_t)page * p.block_size + (t0 % p.block_size);
  }
  const int64_t tok_stride = (int64_t)p.hkv * HD;
  const int64_t head_off = (int64_t)h * HD;

  // Q as the B operand: column n is query head h*G+n, k slot (g, st, j) is d = 32g+8st+j.
  u32x4 qv[4];
  if (n < G) {
    const uint16_t* qr = p.q + (int64_t)b * p.q_stride + (int64_t)(h * G + n) * HD + 32 * g;
#pragma unroll
    for (int st = 0; st < 4; ++st) qv[st] = ld16(qr + 8 * st);
  } else {
#pragma unroll
    for (int st = 0; st < 4; ++st) qv[st] = u32x4{0, 0, 0, 0};
  }

  // K as the A operand: row (token) 16mt+n, same k slots.
  u32x4 ka[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int tok = 16 * mt + n;
    if (tok < ntok) {
      const int64_t e = (slot0 + tok) * tok_stride + head_off + 32 * g;
      if constexpr (FP8) {
        const uint8_t* kr = static_cast<const uint8_t*>(p.k_cache) + e;
        const u32x4 w0 = ld16(kr), w1 = ld16(kr + 16);
        ka[mt][0] = fp8x8_to_bf16x8(u32x2{w0.x, w0.y});
        ka[mt][1] = fp8x8_to_bf16x8(u32x2{w0.z, w0.w});
        ka[mt][2] = fp8x8_to_bf16x8(u32x2{w1.x, w1.y});
        ka[mt][3] = fp8x8_to_bf16x8(u32x2{w1.z, w1.w});
      } else {
        const uint16_t* kr = static_cast<const uint16_t*>(p.k_cache) + e;
#pragma unroll
        for (int st = 0; st < 4; ++st) ka[mt][st] = ld16(kr + 8 * st);
      }
    } else {
#pragma unroll
      for (int st = 0; st < 4; ++st) ka[mt][st] = u32x4{0, 0, 0, 0};
    }
  }

  // V tile -> registers (natural layout): lane covers token 4*it+g, chunk n.
  u32x4 vr[16];
#pragma unroll
  for (int it = 0; it < 16; ++it) {
    const int tok = 4 * it + g;
    if (tok < ntok) {
      const int64_t e = (slot0 + tok) * tok_stride + head_off + 8 * n;
      if constexpr (FP8) vr[it] = fp8x8_to_bf16x8(ld8(static_cast<const uint8_t*>(p.v_cache) + e));
      else vr[it] = ld16(static_cast<const uint16_t*>(p.v_cache) + e);
    } else {
      vr[it] = u32x4{0, 0, 0, 0};
    }
  }

  float ksc[4][4], vsc[4][4];
  if constexpr (FP8) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tok = 16 * mt + 4 * g + i;
        const bool ok = tok < ntok;
        const int64_t si = (slot0 + tok) * p.hkv + h;
        ksc[mt][i] = ok ? p.k_scale[si] : 0.0f;
        vsc[mt][i] = ok ? p.v_scale[si] : 0.0f;
      }
  }

  // S^T = K Q^T for the wavefront's 64 tokens.
  f32x4 s[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    s[mt] = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int st = 0; st < 4; ++st) s[mt] = mfma16(as_bf16x8(ka[mt][st]), as_bf16x8(qv[st]), s[mt]);
  }

  float mx = NEG_INF;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tok = 16 * mt + 4 * g + i;
      float x = s[mt][i] * p.scale_log2;
      if constexpr (FP8) x *= ksc[mt][i];
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
      s[mt][i] = FP8 ? e * vsc[mt][i] : e;
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

  uint16_t* vl = sm.u.dec_v[wave];
#pragma unroll
  for (int it = 0; it < 16; ++it) st16(vl + (4 * it + g) * ROW + 8 * n, vr[it]);
  __syncthreads();

  f32x4 o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = f32x4{0, 0, 0, 0};
  const int src_tok = n >> 2, src_col = 4 * (n & 3);
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const uint16_t* a0 = vl + (32 * ks + 4 * g + src_tok) * ROW + 16 * dt + src_col;
      const bf16x8 vt = join_tr(lds_tr16(a0), lds_tr16(a0 + 16 * ROW));
      o[dt] = mfma16(vt, pb[ks], o[dt]);
    }
  __syncthreads();  // the merge area aliases the V tiles

  if (n < G) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) sm.u.mg.o[wave][n][16 * dt + 4 * g + i] = o[dt][i];
    if (g == 0) {
      sm.u.mg.m[wave][n] = mx;
      sm.u.mg.l[wave][n] = ls;
    }
  }
  __syncthreads();

  float* part = p.partials + (size_t)dindex * G * (HD + 2);
  for (int idx = tid; idx < G * HD; idx += NT) {
    const int hn = idx / HD, d = idx % HD;
    float M = NEG_INF;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, sm.u.mg.m[w][hn]);
    float Ls = 0.0f, O = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float mw = sm.u.mg.m[w][hn];
      const float f = mw == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
      Ls += f * sm.u.mg.l[w][hn];
      O += f * sm.u.mg.o[w][hn][d];
    }
    if (nch == 1) {
      p.out[(int64_t)b * p.out_stride + (int64_t)(h * G + hn) * HD + d] =
          (uint16_t)f32_to_bf16_bits(Ls > 0.0f ? O / Ls : 0.0f);
    } else {
      part[hn * HD + d] = O;
      if (d == 0) {
        part[G * HD + 2 * hn] = M;
        part[G * HD + 2 * hn + 1] = Ls;
      }
    }
  }
  if (nch == 1) return;

  // Split-K: the last chunk of (row, kv head) to finish merges all partials.
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const int ticket = atomicAdd(&p.counters[b * p.hkv + h], 1);
    sm.last = ticket == nch - 1;
  }
  __syncthreads();
  if (!sm.last) return;
  __threadfence();
  const int first = dindex - (c * p.hkv + h);
  for (int idx = tid; idx < G * HD; idx += NT) {
    const int hn = idx / HD, d = idx % HD;
    float M = NEG_INF;
    for (int cc = 0; cc < nch; ++cc) {
      const float* pc = p.partials + (size_t)(first + cc * p.hkv + h) * G * (HD + 2);
      M = fmaxf(M, __builtin_nontemporal_load(pc + G * HD + 2 * hn));
    }
    float Ls = 0.0f, O = 0.0f;
    for (int cc = 0; cc < nch; ++cc) {
      const float* pc = p.partials + (size_t)(first + cc * p.hkv + h) * G * (HD + 2);
      const float mc = __builtin_nontemporal_load(pc + G * HD + 2 * hn);
      const float f = mc == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(mc - M);
      Ls += f * __builtin_nontemporal_load(pc + G * HD + 2 * hn + 1);
      O += f * __builtin_nontemporal_load(pc + hn * HD + d);
    }
    p.out[(int64_t)b * p.out_stride + (int64_t)(h * G + hn) * HD + d] =
        (uint16_t)f32_to_bf16_bits(Ls > 0.0f ? O / Ls : 0.0f);
  }
  if (tid == 0) atomicExch(&p.counters[b * p.hkv + h], 0);
}

// --------------------------------------------------------------- prefill item
template <bool FP8, int NQT>
__device__ void prefill_item(const Params& p, Smem<NQT>& sm, int r, int local) {
  constexpr int BQ = 16 * NQT;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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

  u32x4 qv[NQT][4];
#pragma unroll
  for (int nt = 0; nt < NQT; ++nt) {
    const int pos = q0 + 16 * nt + n;
    if (active && pos < Lq && qrow0 + pos < p.num_q_rows) {
      const uint16_t* qr = p.q + (qrow0 + pos) * p.q_stride + (int64_t)hq * HD + 32 * g;
#pragma unroll
      for (int st = 0; st < 4; ++st) qv[nt][st] = ld16(qr + 8 * st);
    } else {
#pragma unroll
      for (int st = 0; st < 4; ++st) qv[nt][st] = u32x4{0, 0, 0, 0};
    }
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

  const bool src_fp8 = FP8 && paged;
  const int src_tok = n >> 2, src_col = 4 * (n & 3);
  for (int kv0 = 0; kv0 < kend; kv0 += TT) {
    const int ntok = min(TT, kend - kv0);
    bool ok = true;
    int64_t slot0 = 0, base, tstride;
    if (paged) {
      const int page = p.ptab[(int64_t)r * p.ptab_stride + kv0 / p.block_size];
      ok = page >= 0 && page < p.num_blocks;
      slot0 = ok ? (int64_t)page * p.block_size + kv0 % p.block_size : 0;
      tstride = (int64_t)p.hkv * HD;
      base = slot0 * tstride + (int64_t)h * HD;
    } else {
      tstride = p.k_stride;
      base = (int64_t)(k_start + kv0) * p.k_stride + (int64_t)h * HD;
    }
    u32x4 kr[4], vr[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int tok = (tid >> 4) + 16 * it, ch = tid & 15;
      if (ok && tok < ntok) {
        if (src_fp8) {
          const int64_t e = base + tok * tstride + 8 * ch;
          kr[it] = fp8x8_to_bf16x8(ld8(static_cast<const uint8_t*>(p.k_cache) + e));
          vr[it] = fp8x8_to_bf16x8(ld8(static_cast<const uint8_t*>(p.v_cache) + e));
        } else if (paged) {
          const int64_t e = base + tok * tstride + 8 * ch;
          kr[it] = ld16(static_cast<const uint16_t*>(p.k_cache) + e);
          vr[it] = ld16(static_cast<const uint16_t*>(p.v_cache) + e);
        } else {
          const int64_t ek = (int64_t)(k_start + kv0 + tok) * p.k_stride + (int64_t)h * HD + 8 * ch;
          const int64_t ev = (int64_t)(k_start + kv0 + tok) * p.v_stride + (int64_t)h * HD + 8 * ch;
          kr[it] = ld16(p.k + ek);
          vr[it] = ld16(p.v + ev);
        }
      } else {
        kr[it] = u32x4{0, 0, 0, 0};
        vr[it] = u32x4{0, 0, 0, 0};
      }
    }
    float ksv = 1.0f, vsv = 1.0f;
    if (src_fp8 && tid < TT) {
      const bool okt = ok && tid < ntok;
      const int64_t si = (slot0 + tid) * p.hkv + h;
      ksv = okt ? p.k_scale[si] : 0.0f;
      vsv = okt ? p.v_scale[si] : 0.0f;
    }
    __syncthreads();  // previous tile fully consumed
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int tok = (tid >> 4) + 16 * it, ch = tid & 15;
      st16(sm.u.pf.k + tok * ROW + 8 * ch, kr[it]);
      st16(sm.u.pf.v + tok * ROW + 8 * ch, vr[it]);
    }
    if (tid < TT) {
      sm.u.pf.ks[tid] = ksv;
      sm.u.pf.vs[tid] = vsv;
    }
    __syncthreads();
    if (!active) continue;

    f32x4 s[4][NQT];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      u32x4 kf[4];
#pragma unroll
      for (int st = 0; st < 4; ++st) kf[st] = ld16(sm.u.pf.k + (16 * mt + n) * ROW + 32 * g + 8 * st);
#pragma unroll
      for (int nt = 0; nt < NQT; ++nt) {
        f32x4 acc = f32x4{0, 0, 0, 0};
#pragma unroll
        for (int st = 0; st < 4; ++st) acc = mfma16(as_bf16x8(kf[st]), as_bf16x8(qv[nt][st]), acc);
        s[mt][nt] = acc;
      }
    }

    bf16x8 pb[NQT][2];
#pragma unroll
    for (int nt = 0; nt < NQT; ++nt) {
      const int pos = q0 + 16 * nt + n;
      const int lim = pos + prefix;  // last visible key index
      float mx = NEG_INF;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int tok = 16 * mt + 4 * g + i;
          float x = s[mt][nt][i] * p.scale_log2;
          if (src_fp8) x *= sm.u.pf.ks[tok];
          x = (tok < ntok && kv0 + tok <= lim) ? x : NEG_INF;
          s[mt][nt][i] = x;
          mx = fmaxf(mx, x);
        }
      mx = wave_max_xor(mx, 16);
      mx = wave_max_xor(mx, 32);
      const float mnew = fmaxf(m[nt], mx);
      const float mu = mnew == NEG_INF ? 0.0f : mnew;
      const float alpha = __builtin_amdgcn_exp2f(m[nt] - mu);
      float rs = 0.0f;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float e = __builtin_amdgcn_exp2f(s[mt][nt][i] - mu);
          rs += e;
          s[mt][nt][i] = src_fp8 ? e * sm.u.pf.vs[16 * mt + 4 * g + i] : e;
        }
      rs += __shfl_xor(rs, 16, 64);
      rs += __shfl_xor(rs, 32, 64);
      l[nt] = l[nt] * alpha + rs;
      m[nt] = mnew;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) o[dt][nt] *= alpha;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        u32x4 w;
        w.x = pack_bf16x2(s[2 * ks][nt][0], s[2 * ks][nt][1]);
        w.y = pack_bf16x2(s[2 * ks][nt][2], s[2 * ks][nt][3]);
        w.z = pack_bf16x2(s[2 * ks + 1][nt][0], s[2 * ks + 1][nt][1]);
        w.w = pack_bf16x2(s[2 * ks + 1][nt][2], s[2 * ks + 1][nt][3]);
        pb[nt][ks] = as_bf16x8(w);
      }
    }

#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const uint16_t* a0 = sm.u.pf.v + (32 * ks + 4 * g + src_tok) * ROW + 16 * dt + src_col;
        const bf16x8 vt = join_tr(lds_tr16(a0), lds_tr16(a0 + 16 * ROW));
#pragma unroll
        for (int nt = 0; nt < NQT; ++nt) o[dt][nt] = mfma16(vt, pb[nt][ks], o[dt][nt]);
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
template <bool FP8, int NQT>
__global__ void __launch_bounds__(NT, 1) paged_attention_kernel(Params p) {
  __shared__ Smem<NQT> sm;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nrows = p.np + p.nd;

  // Per-row item counts -> exclusive prefix in sm.off (block-wide scan).
  const int per = (nrows + NT - 1) / NT;
  const int r0 = tid * per;
  int local_sum = 0;
  for (int r = r0; r < min(r0 + per, nrows); ++r) local_sum += row_items<NQT>(p, r);
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
    run += row_items<NQT>(p, r);
  }
  if (tid == NT - 1) sm.off[nrows] = run;
  __syncthreads();
  const int total = sm.off[nrows];
  const int decode_base = sm.off[p.np];

  for (;;) {
    if (tid == 0) sm.item = atomicAdd(&p.ctrl[0], 1);
    __syncthreads();
    const int item = sm.item;
    if (item >= total) break;
    for (int r = tid; r < nrows; r += NT)
      if (sm.off[r] <= item && item < sm.off[r + 1]) sm.row = r;
    __syncthreads();
    const int r = sm.row;
    const int local = item - sm.off[r];
    if (r < p.np) prefill_item<FP8, NQT>(p, sm, r, local);
    else decode_item<FP8, NQT>(p, sm, r - p.np, local, item - decode_base);
    __syncthreads();
  }

  if (tid == 0) {
    __threadfence();
    if (atomicAdd(&p.ctrl[1], 1) == (int)gridDim.x - 1) {
      atomicExch(&p.ctrl[0], 0);
      atomicExch(&p.ctrl[1], 0);
    }
  }
}

constexpr int kNQT = 2;  // 16-position column tiles per prefill wavefront

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
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&s.wg_per_cu[0], paged_attention_kernel<false, kNQT>, NT, 0) !=
            hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&s.wg_per_cu[1], paged_attention_kernel<true, kNQT>, NT, 0) !=
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
    return fail(SLO_ERR_UNSUPPORTED, "paged_attention: more than 2048 rows in one launch");
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
      if (!a->k || !a->v || (a->k_row_stride % 8) || (a->v_row_stride % 8) ||
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
  constexpr int BQ = 16 * kNQT;
  int64_t bound = 0;
  if (do_dec) bound += (int64_t)p.nd * ((dec_len_cap + CHUNK - 1) / CHUNK) * p.hkv;
  if (do_pf) {
    const int64_t tq = std::max<int64_t>(0, a->num_q_rows - a->num_decode);
    bound += (tq / BQ + p.np) * p.hkv * p.HG;
  }
  const int64_t slots = (int64_t)ds.cus * ds.wg_per_cu[fp8 ? 1 : 0];
  const int grid = (int)std::max<int64_t>(1, std::min<int64_t>(bound, slots));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (fp8) hipLaunchKernelGGL((paged_attention_kernel<true, kNQT>), dim3(grid), dim3(NT), 0, s, p);
  else hipLaunchKernelGGL((paged_attention_kernel<false, kNQT>), dim3(grid), dim3(NT), 0, s, p);
  return check_launch("paged_attention");
}
