// Achievable read rates on this GPU, for judging the attention kernels'
// rooflines against what the memory system delivers rather than only the
// published 8 TB/s:
//
//  * stream: BYTES read once from HBM (four rotated copies, so no launch finds
//    its bytes in L2 or the memory-side cache), split evenly over the grid,
//    16 bytes per lane per access, 8 accesses in flight per lane, either into
//    VGPRs (global_load_dwordx4, non-temporal) or straight into LDS
//    (global_load_lds_dwordx4) with the default cache policy and with the
//    non-temporal one (the route the decode kernels take);
//  * head slices: the decode kernels' pattern over the same bytes taken as
//    pool rows of 8 kv heads x 256 bytes: each workgroup reads one head's
//    256-byte slice of consecutive rows by non-temporal LDS-DMA (4 rows per
//    instruction, two steps of 16 rows per wavefront in flight), the 8 heads
//    of a row range either on workgroups b, b + 8, ..., b + 56 (one XCD) or
//    on consecutive workgroups (eight XCDs);
//  * tiles: the prefill tile pattern, 64 pool rows x 256 bytes (one kv head's
//    slice of a 2 KiB row) for K and for V per tile, double-buffered into LDS
//    by 512 workgroups; the workgroups of one XCD (b % 8) all read one kv
//    head's slices (1 MiB of K and V), so this is the L2 -> LDS fill rate;
//    then the same with every wavefront also reading the landed tile as a
//    16-position prefill tile's MFMA operands (K: 16 ds_read_b128, V^T: 32
//    ds_read_b64_tr_b16, 32 KiB per wavefront), which share the CU's LDS
//    with the DMA writes.
//
// Usage: read_ceiling [BYTES]   (default 207,417,344: the KV bytes of 24
// decode rows of 256-4096 tokens, 50,639 in all, 8 kv heads x 128 bf16).
// Prints one JSON line; best of 10 launches each (HIP events).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

#define CHECK(x)                                                          \
  do {                                                                    \
    hipError_t e_ = (x);                                                  \
    if (e_ != hipSuccess) {                                               \
      std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));        \
      return 1;                                                           \
    }                                                                     \
  } while (0)

namespace {

constexpr int NT = 256;
constexpr int DEPTH = 8;  // 16-byte accesses in flight per lane
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)p; }

__device__ __forceinline__ void dma16(const void* gp, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gp), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma16_nt(const void* gp, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(gp), "s"(lds) : "memory", "m0");
}

__device__ __forceinline__ uint64_t lds_tr16(const uint8_t* p) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(const_cast<uint8_t*>(p)));
  return __builtin_bit_cast(uint64_t, r);
}

// Workgroup b reads [b * per, (b + 1) * per) of `base` (per: a multiple of 4 KiB).
template <bool LDS, bool NTP = false>
__global__ void __launch_bounds__(NT) stream_kernel(const uint8_t* base, uint64_t per, uint32_t* sink) {
  __shared__ __attribute__((aligned(1024))) uint8_t stage[4 * DEPTH * 1024];
  const int tid = threadIdx.x, wave = tid >> 6;
  const uint8_t* src = base + (uint64_t)blockIdx.x * per + tid * 16;
  const int pieces = (int)(per / (NT * 16));
  u32x4 acc = {0, 0, 0, 0};
  for (int i = 0; i < pieces; i += DEPTH) {
    if constexpr (LDS) {
#pragma unroll
      for (int j = 0; j < DEPTH; ++j)
        if (i + j < pieces) {
          const uint32_t dl = __builtin_amdgcn_readfirstlane(lds_addr(stage + (wave * DEPTH + j) * 1024));
          if constexpr (NTP) dma16_nt(src + (uint64_t)(i + j) * NT * 16, dl);
          else dma16(src + (uint64_t)(i + j) * NT * 16, dl);
        }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else {
      u32x4 v[DEPTH];
#pragma unroll
      for (int j = 0; j < DEPTH; ++j)
        v[j] = i + j < pieces
                   ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + (uint64_t)(i + j) * NT * 16))
                   : u32x4{0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < DEPTH; ++j) acc ^= v[j];
    }
  }
  if constexpr (LDS) {
    __syncthreads();
    acc.x = reinterpret_cast<const uint32_t*>(stage)[tid];
  }
  sink[blockIdx.x * NT + tid] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

// Head slices of 2 KiB rows: workgroup b reads head h's 256 bytes of rows
// [grp * rows_per, (grp + 1) * rows_per).  SPREAD: h = b % 8, grp = b / 8;
// otherwise h = (b / 8) % 8, grp = (b / 64) * 8 + b % 8.
template <bool SPREAD>
__global__ void __launch_bounds__(NT) slice_kernel(const uint8_t* base, int rows_per, uint32_t* sink) {
  __shared__ __attribute__((aligned(1024))) uint8_t stage[2][4][4096];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, b = blockIdx.x;
  const int h = SPREAD ? b % 8 : (b / 8) % 8;
  const int grp = SPREAD ? b / 8 : (b / 64) * 8 + b % 8;
  const uint8_t* rows = base + (uint64_t)grp * rows_per * 2048 + 256 * h;
  const int g = lane >> 4, n = lane & 15;
  for (int s = 0; s < rows_per / 64; ++s) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = s * 64 + wave * 16 + 4 * i + g;
      dma16_nt(rows + (uint64_t)r * 2048 + 16 * n,
               __builtin_amdgcn_readfirstlane(lds_addr(stage[s & 1][wave] + 1024 * i)));
    }
    asm volatile("s_waitcnt vmcnt(4)" ::: "memory");  // step s - 1 landed, step s in flight
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  sink[b * NT + tid] = reinterpret_cast<const uint32_t*>(stage)[tid];
}

// Tile t of workgroup b: pool rows 64 * ((t + b / 8) % (rows / 64)) onwards,
// kv head b % 8; K rows at `pool`, V rows `rows` rows later.  READS: every
// wavefront reads the landed tile's K (first 16 KiB) and V (last 16 KiB).
template <bool READS>
__global__ void __launch_bounds__(NT) tile_kernel(const uint8_t* pool, int rows, int ntiles, uint32_t* sink) {
  __shared__ __attribute__((aligned(1024))) uint8_t buf[2 * 32768];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  u32x4 acc = {0, 0, 0, 0};
  uint64_t acc2 = 0;
  const int h = blockIdx.x % 8, nrt = rows / 64;
  auto issue = [&](int t, int b) {
    const int tr = (t + (int)(blockIdx.x / 8)) % nrt;
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int row = (tid >> 4) + 16 * (it & 3);
      const uint8_t* src = pool + (uint64_t)(tr * 64 + row) * 2048 + h * 256 + (tid & 15) * 16 +
                           (it >= 4 ? (uint64_t)rows * 2048 : 0);
      dma16(src, __builtin_amdgcn_readfirstlane(lds_addr(buf + b * 32768 + it * 4096 + wave * 1024)));
    }
  };
  issue(0, 0);
  for (int t = 0; t < ntiles; ++t) {
    if (t + 1 < ntiles) {
      issue(t + 1, (t + 1) & 1);
      asm volatile("s_waitcnt vmcnt(8)" ::: "memory");  // tile t landed, t + 1 in flight
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
    if constexpr (READS) {
      const uint8_t* kt = buf + (t & 1) * 32768;
      // K: lane reads 16 bytes of row (lane & 15) + 16 * (i & 3), chunk ((lane >> 4) + 4 * (i >> 2)) ^ (lane & 15)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        acc ^= *reinterpret_cast<const u32x4*>(kt + ((lane & 15) + 16 * (i & 3)) * 256 +
                                               ((((lane >> 4) + 4 * (i >> 2)) ^ (lane & 15)) & 15) * 16);
      // V^T: transposed 8-byte reads over the V rows
#pragma unroll
      for (int i = 0; i < 32; ++i)
        acc2 ^= lds_tr16(kt + 16384 + ((lane & 15) + 16 * (i & 3)) * 256 +
                         ((((lane >> 4) * 2 + 8 * ((i >> 2) & 1)) ^ ((lane & 7) << 1)) * 8) % 256);
      __syncthreads();  // reads done before the next DMA into this buffer
    }
  }
  sink[blockIdx.x * NT + tid] = reinterpret_cast<const uint32_t*>(buf)[tid] ^ acc.x ^ acc.y ^ acc.z ^ acc.w ^
                                (uint32_t)acc2 ^ (uint32_t)(acc2 >> 32);
}

}  // namespace

int main(int argc, char** argv) {
  const uint64_t want = argc > 1 ? std::strtoull(argv[1], nullptr, 10) : 207417344ull;
  const int grid = 512;  // two workgroups per CU on 256 CUs
  const uint64_t per = want / grid > 4096 ? (want / grid + 4095) / 4096 * 4096 : 4096;
  const uint64_t copy = per * grid;  // bytes one stream launch reads
  const uint64_t copy_stride = (copy + (1 << 20) - 1) >> 20 << 20;
  const int rows = 2048, ntiles = 64;  // tiles: 2 x 4 MiB pool, 512 x 64 tiles of 32 KiB
  const uint64_t pool_bytes = 2ull * rows * 2048;
  uint8_t* buf = nullptr;
  uint32_t* sink = nullptr;
  const uint64_t total = 4 * copy_stride > pool_bytes ? 4 * copy_stride : pool_bytes;
  CHECK(hipMalloc(&buf, total));
  CHECK(hipMalloc(&sink, (size_t)grid * NT * sizeof(uint32_t)));
  CHECK(hipMemset(buf, 1, total));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  // Head slices: 64 row ranges of rows_per 2 KiB rows within one copy.
  const int rows_per = (int)(copy / 2048 / 64 / 64 * 64);
  const double slices = (double)grid * rows_per * 256;
  double best[7] = {1e30, 1e30, 1e30, 1e30, 1e30, 1e30, 1e30};
  for (int kind = 0; kind < 7; ++kind) {
    for (int rep = 0; rep < 12; ++rep) {
      const uint8_t* base = buf + (uint64_t)(rep % 4) * copy_stride;
      CHECK(hipEventRecord(e0));
      if (kind == 0) stream_kernel<false><<<grid, NT>>>(base, per, sink);
      else if (kind == 1) stream_kernel<true><<<grid, NT>>>(base, per, sink);
      else if (kind == 2) tile_kernel<false><<<grid, NT>>>(buf, rows, ntiles, sink);
      else if (kind == 3) tile_kernel<true><<<grid, NT>>>(buf, rows, ntiles, sink);
      else if (kind == 4) stream_kernel<true, true><<<grid, NT>>>(base, per, sink);
      else if (kind == 5) slice_kernel<false><<<grid, NT>>>(base, rows_per, sink);
      else slice_kernel<true><<<grid, NT>>>(base, rows_per, sink);
      CHECK(hipEventRecord(e1));
      CHECK(hipEventSynchronize(e1));
      float ms = 0.0f;
      CHECK(hipEventElapsedTime(&ms, e0, e1));
      if (rep >= 2 && ms < best[kind]) best[kind] = ms;  // two warm-up launches
    }
  }
  CHECK(hipGetLastError());
  const double tiles = (double)grid * ntiles * 32768;
  std::printf(
      "{\"bytes\": %llu, \"stream_vgpr_us\": %.2f, \"stream_vgpr_TBps\": %.3f, \"stream_lds_dma_us\": %.2f, "
      "\"stream_lds_dma_TBps\": %.3f, \"stream_lds_dma_nt_us\": %.2f, \"stream_lds_dma_nt_TBps\": %.3f, "
      "\"head_slice_bytes\": %.0f, \"head_slices_one_xcd_us\": %.2f, \"head_slices_one_xcd_TBps\": %.3f, "
      "\"head_slices_spread_us\": %.2f, \"head_slices_spread_TBps\": %.3f, "
      "\"tile_fill_TBps\": %.2f, \"tile_us_per_workgroup\": %.3f, "
      "\"tile_fill_with_operand_reads_TBps\": %.2f, \"tile_with_operand_reads_us_per_workgroup\": %.3f}\n",
      (unsigned long long)copy, best[0] * 1e3, copy / (best[0] * 1e-3) / 1e12, best[1] * 1e3,
      copy / (best[1] * 1e-3) / 1e12, best[4] * 1e3, copy / (best[4] * 1e-3) / 1e12, slices, best[5] * 1e3,
      slices / (best[5] * 1e-3) / 1e12, best[6] * 1e3, slices / (best[6] * 1e-3) / 1e12,
      tiles / (best[2] * 1e-3) / 1e12, best[2] * 1e3 / ntiles, tiles / (best[3] * 1e-3) / 1e12,
      best[3] * 1e3 / ntiles);
  return 0;
}
