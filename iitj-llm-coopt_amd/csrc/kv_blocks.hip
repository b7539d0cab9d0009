// Block migration copy for the paged KV pool (engine/block_manager.py:165-187, whose copy_fn
// is `buf[dst].copy_(buf[src])` at engine/elastic.py:131).  The reference issues one torch
// copy per migrated block; here every (src, dst) pair of a migration, in every cache region,
// is one launch (or one per 32 regions).
//
// A region is any tensor whose blocks are dense byte ranges at a fixed stride: the whole
// block-major elastic buffer [NB, L, 2, bs, Hkv, D] (one 2 MiB block per id for the 8B
// target), or one per-layer K / V cache or INT8 scale cache.  The work is a pure HBM copy:
// workgroups stream 32 KiB chunks, eight independent 16-byte loads per lane in flight
// before the stores, consecutive workgroups on consecutive chunks of one block.  Loads and
// stores are nontemporal (nothing is reused); on MI355X that moves 256 x 2 MiB blocks at
// 5.8 TB/s against 5.3 TB/s with ordinary accesses.
#include "common.h"

namespace {

constexpr int kMaxRegions = 32;   // regions per launch (passed by value in the kernel args)
constexpr int kThreads = 256;
constexpr int kVecPerThread = 8;  // 16-byte vectors per lane per chunk
constexpr int64_t kChunk = int64_t(kThreads) * kVecPerThread * 16;  // 32 KiB

// 16-byte vectors in the global address space (the bases arrive as integers, so the
// compiler would otherwise emit flat accesses).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) u32x4 gvec;

struct Region {
  int64_t base;    // device address
  int64_t stride;  // bytes between consecutive block ids
  int64_t bytes;   // bytes per block (multiple of 16)
};

struct RegionSet {
  Region r[kMaxRegions];
  int n;
  int chunks;      // chunks per (pair, region): ceil(max bytes / kChunk)
};

// grid.x = num_pairs * set.n * set.chunks; blockIdx -> (pair, region, chunk), chunk fastest.
__global__ __launch_bounds__(kThreads) void copy_blocks_kernel(
    RegionSet set, const int64_t* __restrict__ src_ids, const int64_t* __restrict__ dst_ids,
    int64_t num_blocks) {
  // the host keeps grid * kThreads < 2^32, so 32-bit division suffices
  const uint32_t wg = blockIdx.x;
  const uint32_t chunk = wg % static_cast<uint32_t>(set.chunks);
  const uint32_t rest = wg / static_cast<uint32_t>(set.chunks);
  const uint32_t reg = rest % static_cast<uint32_t>(set.n);
  const uint32_t pair = rest / static_cast<uint32_t>(set.n);
  const int64_t s = src_ids[pair], d = dst_ids[pair];
  if (s < 0 || s >= num_blocks || d < 0 || d >= num_blocks) return;
  const Region R = set.r[reg];
  const int64_t begin = int64_t(chunk) * kChunk;
  if (begin >= R.bytes) return;
  const int64_t from = R.base + s * R.stride + begin;
  const int64_t to = R.base + d * R.stride + begin;
  const int64_t left = R.bytes - begin;
  const gvec* f = reinterpret_cast<const gvec*>(from) + threadIdx.x;
  gvec* t = reinterpret_cast<gvec*>(to) + threadIdx.x;
  if (left >= kChunk) {  // whole chunk: every load in flight before the first store
    u32x4 v[kVecPerThread];
#pragma unroll
    for (int i = 0; i < kVecPerThread; ++i) v[i] = __builtin_nontemporal_load(f + i * kThreads);
#pragma unroll
    for (int i = 0; i < kVecPerThread; ++i) __builtin_nontemporal_store(v[i], t + i * kThreads);
  } else {               // the block's tail (or a block smaller than a chunk)
    const int n = static_cast<int>(left / 16);
    for (int i = threadIdx.x; i < n; i += kThreads) t[i - threadIdx.x] = f[i - threadIdx.x];
  }
}

}  // namespace

extern "C" int coopt_kv_copy_blocks(const int64_t* regions, int num_regions,
                                    const int64_t* src_ids, const int64_t* dst_ids,
                                    int num_pairs, int64_t num_blocks, coopt_stream_t stream) {
  coopt::clear_error();
  COOPT_REQUIRE(num_regions >= 0 && num_pairs >= 0 && num_blocks >= 0, "negative count");
  if (num_regions == 0 || num_pairs == 0) return COOPT_OK;
  COOPT_REQUIRE(regions != nullptr, "null region table");
  COOPT_REQUIRE(src_ids != nullptr && dst_ids != nullptr, "null block id array");
  for (int i = 0; i < num_regions; ++i) {
    const int64_t base = regions[3 * i], stride = regions[3 * i + 1], bytes = regions[3 * i + 2];
    COOPT_REQUIRE(base != 0, "region " + std::to_string(i) + ": null base");
    COOPT_REQUIRE(((base | stride | bytes) & 15) == 0,
                  "region " + std::to_string(i) + ": base, block stride and bytes per block "
                  "must be multiples of 16");
    COOPT_REQUIRE(bytes > 0 && bytes <= stride,
                  "region " + std::to_string(i) + ": bytes per block must be in (0, block stride]");
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  for (int r0 = 0; r0 < num_regions; r0 += kMaxRegions) {
    RegionSet set{};
    set.n = num_regions - r0 < kMaxRegions ? num_regions - r0 : kMaxRegions;
    int64_t max_bytes = 0;
    for (int i = 0; i < set.n; ++i) {
      const int64_t* t = regions + 3 * (r0 + i);
      set.r[i] = Region{t[0], t[1], t[2]};
      max_bytes = t[2] > max_bytes ? t[2] : max_bytes;
    }
    const int64_t chunks = (max_bytes + kChunk - 1) / kChunk;
    const int64_t grid = int64_t(num_pairs) * set.n * chunks;
    // the launch's thread count in x (grid * kThreads) must fit 32 bits
    COOPT_REQUIRE(grid * kThreads <= int64_t(0xffffffff), "migration too large for one launch");
    set.chunks = static_cast<int>(chunks);
    hipLaunchKernelGGL(copy_blocks_kernel, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0,
                       s, set, src_ids, dst_ids, num_blocks);
    const int rc = coopt::check_launch("coopt_kv_copy_blocks");
    if (rc != COOPT_OK) return rc;
  }
  return COOPT_OK;
}

// ---------------------------------------------------------------------------------------
// Paged addressing of a batch of row runs, on the device: sequence b owns rows
// [b * S, (b + 1) * S) at positions start[b] + j, with cache slot
// table[b][p / bs] * bs + p % bs (engine/block_manager.py:216-220) and seq_len start[b] + S
// (engine/batch.py:23-55; the padded layout of engine/cuda_graphs.py:76-104).  Rows with
// j >= n_real[b] (padding) or a block index outside [0, table_width) get slot -1: the KV
// write skips them.
// ---------------------------------------------------------------------------------------
namespace {

__global__ __launch_bounds__(kThreads) void row_slots_kernel(
    const int32_t* __restrict__ table, int64_t table_stride, int width,
    const int64_t* __restrict__ start, const int64_t* __restrict__ n_real, int B, int S, int bs,
    int64_t* __restrict__ pos_out, int64_t* __restrict__ slot_out, int32_t* __restrict__ seq_lens) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (gid >= static_cast<int64_t>(B) * S) return;
  const int b = static_cast<int>(gid / S), j = static_cast<int>(gid - static_cast<int64_t>(b) * S);
  const int64_t s0 = start[b];
  const int64_t p = s0 + j;
  const int64_t blk = p >= 0 ? p / bs : -1;
  const bool real = n_real == nullptr || j < n_real[b];
  int64_t slot = -1;
  if (real && blk >= 0 && blk < width)
    slot = static_cast<int64_t>(table[b * table_stride + blk]) * bs + (p - blk * bs);
  pos_out[gid] = p;
  slot_out[gid] = slot;
  if (j == 0 && seq_lens != nullptr) seq_lens[b] = static_cast<int32_t>(s0 + S);
}

}  // namespace

extern "C" int coopt_row_slots(const int32_t* block_table, int64_t table_stride, int table_width,
                               const int64_t* start, const int64_t* n_real, int B, int S,
                               int block_size, int64_t* positions, int64_t* slots,
                               int32_t* seq_lens, coopt_stream_t stream) {
  coopt::clear_error();
  COOPT_REQUIRE(B >= 0 && S >= 0, "negative size");
  if (B == 0 || S == 0) return COOPT_OK;
  COOPT_REQUIRE(block_table && start && positions && slots, "null pointer");
  COOPT_REQUIRE(block_size > 0 && table_width > 0 && table_stride >= table_width,
                "block_size and table_width must be positive, table_stride >= table_width");
  const int64_t n = static_cast<int64_t>(B) * S;
  COOPT_REQUIRE((n + kThreads - 1) / kThreads <= 0x7fffffff, "too many rows");
  hipLaunchKernelGGL(row_slots_kernel, dim3(static_cast<unsigned>((n + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, reinterpret_cast<hipStream_t>(stream), block_table,
                     table_stride, table_width, start, n_real, B, S, block_size, positions, slots,
                     seq_lens);
  return coopt::check_launch("coopt_row_slots");
}
