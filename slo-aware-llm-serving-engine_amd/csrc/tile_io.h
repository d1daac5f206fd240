// LDS tile addressing, LDS-DMA and memory-operation helpers shared by the
// attention kernels (gfx950).  Layout facts the swizzles and the transposing
// read rely on are listed in common.h.
#pragma once
#include "common.h"

namespace slo {

constexpr int HD = 128;          // head_dim the attention kernels implement
constexpr int ROWB = HD * 2;     // bytes of one bf16 K or V row of one kv head

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
// v_max_f32 without the canonicalising max(x, x) the compiler puts on each
// operand of fmaxf that comes out of a lane swap (the scores are never NaN:
// masked ones are -inf by selection).
__device__ __forceinline__ float vmax(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float col_max(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = vmax(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmax(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float col_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// s_waitcnt immediate that waits for vmcnt <= n and nothing else (gfx9 encoding).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// LDS byte address of a pointer into a __shared__ array (wave-uniform).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p);
}

// global -> LDS DMA: lane i's 16 (or 4) bytes at gp land at LDS lds + 16i (4i).
__device__ __forceinline__ void dma16(const void* gp, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gp), "s"(lds) : "memory", "m0");
}
// The same with the non-temporal cache policy, for bytes read exactly once
// (the decode K/V stream: every 128-byte line is read whole by one
// instruction).  A pass over 207.6 MB reads at 6.7 TB/s this way against 5.6
// TB/s with the default policy; data that other workgroups read again (the
// prefill tiles) keeps the default.
__device__ __forceinline__ void dma16_nt(const void* gp, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(gp), "s"(lds) : "memory", "m0");
}
// The same from a wave-uniform base plus a 32-bit per-lane byte offset (the
// saddr form: the base stays in SGPRs, so a tile's loads need no per-lane
// 64-bit address arithmetic).
__device__ __forceinline__ void dma16_at(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds)
               : "memory", "m0");
}
// Four LDS-DMA loads that fill 4 KiB of LDS from one M0 write: load i lands
// at lds + 1024 i and reads base + o[i] + 1024 i (the instruction offset is
// added to the global and the LDS address alike), so the caller passes o[i]
// already lowered by 1024 i.  One M0 write and one wait state for four loads.
__device__ __forceinline__ void dma16x4_at(const void* base, const int (&o)[4], uint32_t lds) {
  asm volatile(
      "s_mov_b32 m0, %5\n\ts_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %4\n\t"
      "global_load_lds_dwordx4 %1, %4 offset:1024\n\t"
      "global_load_lds_dwordx4 %2, %4 offset:2048\n\t"
      "global_load_lds_dwordx4 %3, %4 offset:3072" ::"v"(o[0]),
      "v"(o[1]), "v"(o[2]), "v"(o[3]), "s"(base), "s"(lds)
      : "memory", "m0");
}
// The same with 64-bit lane addresses (p_i already lowered by 1024 i bytes).
__device__ __forceinline__ void dma16x4(const void* p0, const void* p1, const void* p2, const void* p3,
                                        uint32_t lds) {
  asm volatile(
      "s_mov_b32 m0, %4\n\ts_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off\n\t"
      "global_load_lds_dwordx4 %1, off offset:1024\n\t"
      "global_load_lds_dwordx4 %2, off offset:2048\n\t"
      "global_load_lds_dwordx4 %3, off offset:3072" ::"v"(p0),
      "v"(p1), "v"(p2), "v"(p3), "s"(lds)
      : "memory", "m0");
}
// A pointer that is the same in every lane, moved to SGPRs.
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  return (const void*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ void dma4(const void* gp, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(gp), "s"(lds) : "memory", "m0");
}
// Atomic add returning the old value; the value is valid only after a wait
// that covers this operation.
__device__ __forceinline__ uint32_t atomic_add_ret(void* p, uint32_t v) {
  uint32_t r;
  asm volatile("global_atomic_add %0, %1, %2, off sc0" : "=v"(r) : "v"(p), "v"(v) : "memory");
  return r;
}
__device__ __forceinline__ void atomic_add_noret(void* p, uint32_t v) {
  asm volatile("global_atomic_add %0, %1, off" ::"v"(p), "v"(v) : "memory");
}
// Stores: agent-scope (write-through to the coherence point) for split-K
// partials, plain for outputs.
__device__ __forceinline__ void store16_agent(void* p, const u32x4& v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store16(void* p, const u32x4& v) {
  asm volatile("global_store_dwordx4 %0, %1, off" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store8(void* p, const u32x2& v) {
  asm volatile("global_store_dwordx2 %0, %1, off" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store8_agent(void* p, const u32x2& v) {
  asm volatile("global_store_dwordx2 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store4(void* p, uint32_t v) {
  asm volatile("global_store_dword %0, %1, off" ::"v"(p), "v"(v) : "memory");
}
// Ties x to this point: uses of x cannot move above an earlier wait.
__device__ __forceinline__ uint32_t after_wait(uint32_t x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Workgroup barrier that orders LDS accesses only.  __syncthreads() also waits
// for every LDS DMA write still in flight (vmcnt), which would drain the KV
// loads; the decode stages are private to their wavefront, so the barriers of
// the decode loop (Q, merge area, item broadcast) need only the LDS counter.
// The empty asm statements keep the compiler from moving memory accesses
// across the barrier.
__device__ __forceinline__ void lds_sync() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace slo
