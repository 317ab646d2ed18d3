// Batched decode attention for callers that cannot allocate device memory:
// pa_decode_batched_noalloc_f16 runs the same kernels as pa_decode_batched_f16,
// with the split-K scratch (pair counters and partial records) in a fixed
// array owned by the library instead of a caller's workspace.
//
// The array, `scratch`, is a file-scope __device__ variable: every GPU the
// library runs on holds its own copy, at its own address, until the process
// ends. Host code never passes the array's name to a kernel (on the host it is
// only a stand-in for the symbol): the first call on each device looks up that
// device's address with hipGetSymbolAddress, with the device current, and
// keeps it; every launch then takes that address. The same first call clears
// the counter region with a fill kernel on the call's stream (not a memset,
// so the call may sit inside a captured graph); each completed call leaves the
// counters zero again, as the kernel's protocol requires.
#include <mutex>

#include "../../include/paged_attention.h"
#include "pa_common.h"

namespace pa {

// Counters (kSkCounterBytes) plus two partial records per workgroup of a
// 256-CU grid at head_dim 256 (8.5 MB) fit with room to spare.
constexpr size_t kNoAllocScratchBytes = PA_NOALLOC_SCRATCH_BYTES;
static_assert(kNoAllocScratchBytes > kSkCounterBytes, "scratch holds the counter region");

static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mutex;
void* g_scratch[kMaxDevices];  // device address of `scratch` per device, once looked up

__global__ void clear_words(int* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

// Device address of this device's `scratch`; set up on the device's first call.
int scratch_address(void** ptr, hipStream_t stream) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("no usable current HIP device (%s)", hipGetErrorString(e));
    return PA_ERR_HIP;
  }
  std::lock_guard<std::mutex> lock(g_mutex);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("hipGetSymbolAddress of the decode scratch failed on device %d: %s", dev,
                hipGetErrorString(e));
      return PA_ERR_HIP;
    }
    constexpr int words = (int)(kSkCounterBytes / sizeof(int));
    clear_words<<<64, 256, 0, stream>>>(static_cast<int*>(p), words);
    e = hipGetLastError();
    if (e != hipSuccess) {
      set_error("clearing the decode scratch failed on device %d: %s", dev, hipGetErrorString(e));
      return PA_ERR_HIP;
    }
    g_scratch[dev] = p;
  }
  *ptr = g_scratch[dev];
  return PA_OK;
}

}  // namespace
}  // namespace pa

extern "C" {

int pa_decode_batched_noalloc_f16(const void* q, const int64_t q_strides[3], const void* k_cache,
                                  const int64_t k_strides[4], const void* v_cache,
                                  const int64_t v_strides[4], const int32_t* block_tables,
                                  const int64_t bt_strides[2], const int32_t* seq_lens,
                                  void* out, const int64_t out_strides[3], int num_seqs,
                                  int num_q_heads, int num_kv_heads, int head_dim,
                                  int block_size, int num_blocks, int max_blocks_per_seq,
                                  float scale, void* stream) {
  pa::clear_error();
  return pa::decode_batched(q, q_strides, k_cache, k_strides, v_cache, v_strides, block_tables,
                            bt_strides, seq_lens, out, out_strides, num_seqs, num_q_heads,
                            num_kv_heads, head_dim, block_size, num_blocks, max_blocks_per_seq,
                            scale, nullptr, pa::kNoAllocScratchBytes, pa::scratch_address, stream);
}

}  // extern "C"
