// Device helpers shared by the gfx950 decode-attention kernels: tile loads,
// LDS access patterns, coherent partial records.
#pragma once

#include "pa_common.h"

namespace pa {
namespace tiles {

constexpr int kXcds = 8;  // accelerator complex dies of an MI355X, each with its own L2

__device__ inline f16x8 zero8() { return f16x8{0, 0, 0, 0, 0, 0, 0, 0}; }

// K/V register buffers hold raw 16-byte pieces as 32-bit lanes: kept as fp16
// vectors, the compiler merges a buffer array into one wide half vector and
// splices new loads into it with half-word bit inserts, which must wait for
// the loads at the splice instead of at the use.
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Orders one wavefront's LDS writes before its later LDS reads (and reads
// before later writes). LDS instructions of a wavefront execute in order, so
// only the compiler has to be kept from moving them.
__device__ inline void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// K/V rows are read with the non-temporal hint (global_load_dwordx4 ... nt):
// measured on MI355X, random 4 KB block gathers reach ~6.6 TB/s with it
// against ~5.9 TB/s with default-policy loads.
__device__ inline u32x4 load_stream(const f16* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Buffer resource over `bytes` bytes at a wavefront-uniform base. Loads at
// offsets past `bytes` return zeros and touch no memory, so a load of a tile
// past the end of the work is issued with bytes = 0 instead of being skipped:
// the loop then has no branches around its loads, and the compiler's count of
// loads in flight stays exact (a skipped load on one path would force every
// wait to assume the shorter path and drain the pipeline).
__device__ inline __amdgpu_buffer_rsrc_t tile_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// 16-byte K/V load through a tile resource: per-lane offset plus a uniform
// offset, cache policy sc0 | nt (stream past the L1, non-temporal in L2) --
// measured on MI355X at ~6.6 TB/s for random 4 KB block gathers.
__device__ inline u32x4 load_tile(__amdgpu_buffer_rsrc_t r, uint32_t lane_off, int uoff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)lane_off, uoff, 3);
}

// Transposing LDS read (ds_read_b64_tr_b16): within each group of 16 lanes,
// lane 4 r + q supplies the address of halves [4 q, 4 q + 4) of row r of a
// 4 x 16 block, and lane j receives column j of that block (rows 0..3).
__device__ inline f16x4 lds_read_tr16(const f16* p) {
  typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 v4h;
  auto* lp = (__attribute__((address_space(3))) v4h*)(const_cast<f16*>(p));
  return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16(lp));
}

// Partial records cross XCDs (each has its own L2): they are written and read
// with device-coherent accesses (agent-scope atomic stores and loads: sc1
// write-through / coherent-miss), so publishing one needs no L2 writeback or
// invalidate -- fences that would stall the whole XCD's L2 mid-kernel.
__device__ inline void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float load_coherent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 16-byte forms of the same device-coherent accesses, through a buffer
// resource (cache policy sc1, the bit the agent-scope stores and loads above
// carry). Unlike atomic loads, the compiler issues many of these before
// waiting, so reading a record costs one memory round trip.
__device__ inline void store_coherent16(__amdgpu_buffer_rsrc_t r, int byte_off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, byte_off, 0, 16);
}
__device__ inline f32x4 load_coherent16(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 16));
}
__device__ inline float load_coherent4(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 16));
}

// Read of a table entry at a wavefront-uniform address through the scalar
// data cache (s_load): the block tables and lengths are never written by
// these kernels, and scalar loads are counted apart from the vector loads, so
// waiting for a block id never waits for the K/V loads issued before it.
__device__ inline int load_uniform(const int32_t* p) {
  return *(const __attribute__((address_space(4))) int32_t*)p;
}

template <int BS>
__device__ inline int blk_of(int t, int bs) {
  if constexpr (BS > 0) return t / BS; else return t / bs;
}

template <int BS>
__device__ inline int off_of(int t, int bs) {
  if constexpr (BS > 0) return t % BS; else return t % bs;
}

}  // namespace tiles
}  // namespace pa
