// Read-bandwidth probes of the benchmark: the practical HBM read ceilings on
// the box the decode kernel is measured on. Measurement infrastructure only;
// nothing in the attention path calls them. Declarations: include/bw_probe.h.
//
// bwp_read_stream: every byte of a buffer read once with 16-byte loads, each
//   load instruction of a wavefront covering 1 KB contiguous (whole cache
//   lines), the same non-temporal buffer-load policy as the decode kernel's
//   K/V loads.
// bwp_gather_blocks: a list of blocks of a pool (the K/V blocks of a paged
//   pool) read in list order, one block per wavefront step, four blocks in
//   flight per wavefront (as many bytes as a decode wavefront keeps in flight),
//   again with the decode kernel's load instruction.
#include "../csrc/pa_tiles.h"
#include "../../include/bw_probe.h"

namespace {

using namespace pa;
using namespace pa::tiles;

constexpr int kThreads = 512;
constexpr int kUnroll = 16;  // 16-byte loads in flight per lane (16 KB per wavefront)
constexpr int kGatherBlocks = 4;  // blocks in flight per wavefront

__global__ __launch_bounds__(kThreads) void read_stream_kernel(const char* buf, int64_t bytes,
                                                               unsigned* sink) {
  const int lane = threadIdx.x & 63;
  const int64_t waves = (int64_t)gridDim.x * (kThreads / 64);
  const int64_t wave = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  // A wavefront step reads kUnroll KB: instruction u covers bytes [u KB, u KB + 1 KB).
  constexpr int64_t kStep = 1024 * kUnroll;
  const int64_t steps = bytes / kStep;
  u32x4 acc = {0, 0, 0, 0};
  for (int64_t s = wave; s < steps; s += waves) {
    const auto r = tile_rsrc(buf + s * kStep, (int)kStep);
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = load_tile(r, lane * 16, u * 1024);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= v[u];
  }
  const unsigned x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (x == 0x9e3779b9u) sink[0] = x;  // keeps the loads; practically never taken
}

__global__ __launch_bounds__(kThreads) void gather_kernel(const char* pool, const int32_t* ids,
                                                          int n_ids, int block_bytes,
                                                          int num_blocks, unsigned* sink) {
  const int lane = threadIdx.x & 63;
  const int waves = gridDim.x * (kThreads / 64);
  const int wave = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  const int per = block_bytes / 1024;  // 1 KB load instructions per block (at most 4)
  u32x4 acc = {0, 0, 0, 0};
  for (int i = wave; i < n_ids; i += kGatherBlocks * waves) {
    u32x4 v[kGatherBlocks][4];
#pragma unroll
    for (int k = 0; k < kGatherBlocks; ++k) {
      const int j = i + k * waves;
      int id = 0;
      if (j < n_ids) id = min(max(__builtin_amdgcn_readfirstlane(ids[j]), 0), num_blocks - 1);
      const auto r = tile_rsrc(pool + (int64_t)id * block_bytes, j < n_ids ? block_bytes : 0);
#pragma unroll
      for (int u = 0; u < 4; ++u) v[k][u] = load_tile(r, lane * 16, u < per ? u * 1024 : 0x7ffffff0);
    }
#pragma unroll
    for (int k = 0; k < kGatherBlocks; ++k)
#pragma unroll
      for (int u = 0; u < 4; ++u) acc ^= v[k][u];
  }
  const unsigned x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (x == 0x9e3779b9u) sink[0] = x;
}

}  // namespace

extern "C" {

int bwp_read_stream(const void* buf, int64_t bytes, void* sink, int grid, void* stream) {
  if (!buf || !sink || bytes <= 0 || grid <= 0 || ((uintptr_t)buf & 15)) return 1;
  read_stream_kernel<<<grid, kThreads, 0, (hipStream_t)stream>>>((const char*)buf, bytes,
                                                                  (unsigned*)sink);
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

int bwp_gather_blocks(const void* pool, int num_blocks, int block_bytes, const int32_t* ids,
                      int n_ids, void* sink, int grid, void* stream) {
  if (!pool || !ids || !sink || num_blocks <= 0 || n_ids <= 0 || grid <= 0 ||
      block_bytes <= 0 || block_bytes > 4096 || block_bytes % 1024 || ((uintptr_t)pool & 15))
    return 1;
  gather_kernel<<<grid, kThreads, 0, (hipStream_t)stream>>>((const char*)pool, ids, n_ids,
                                                             block_bytes, num_blocks,
                                                             (unsigned*)sink);
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

}  // extern "C"
