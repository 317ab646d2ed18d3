// Per-step K/V write into the paged pool (gfx950).
//
// Semantics follow paged_decode_attention_forward,
// engine/kernels/paged_attention_integration.py:148-161: for sequence b with
// L = seq_lens[b], the new token sits at position L-1, i.e. logical block
// (L-1) / block_size, row (L-1) % block_size; all kv heads of key[b] and
// value[b] are copied there. The copy moves 16-bit patterns (no float
// conversion), so the pool receives the exact bits of key/value.
// One thread copies one 16-byte slice when both sources have unit head_dim
// stride and 16-byte aligned rows, one element otherwise.
#include "pa_common.h"

namespace pa {

template <bool VEC>
__global__ __launch_bounds__(256) void kv_write_kernel(KVWriteArgs a) {
  const int per_row = VEC ? a.D / 8 : a.D;
  const int64_t total = (int64_t)a.num_seqs * a.hkv * per_row;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(i % per_row);
    const int64_t r = i / per_row;
    const int h = (int)(r % a.hkv);
    const int b = (int)(r / a.hkv);
    const int L = a.lens ? a.lens[b] : a.uniform_len;
    if (L <= 0) continue;
    const int pos = L - 1;
    const int lb = pos / a.bs;
    if (lb >= a.max_blocks) continue;
    const int id = a.bt[(int64_t)b * a.bt_sb + (int64_t)lb * a.bt_sk];
    if (id < 0 || id >= a.num_blocks) continue;
    const int off = pos - lb * a.bs;
    const int64_t dk = (int64_t)id * a.kc_sb + (int64_t)off * a.kc_st + (int64_t)h * a.kc_sh;
    const int64_t dv = (int64_t)id * a.vc_sb + (int64_t)off * a.vc_st + (int64_t)h * a.vc_sh;
    const int64_t sk = (int64_t)b * a.ks_b + (int64_t)h * a.ks_h;
    const int64_t sv = (int64_t)b * a.vs_b + (int64_t)h * a.vs_h;
    if constexpr (VEC) {
      *reinterpret_cast<uint4*>(a.kc + dk + c * 8) = *reinterpret_cast<const uint4*>(a.key + sk + c * 8);
      *reinterpret_cast<uint4*>(a.vc + dv + c * 8) = *reinterpret_cast<const uint4*>(a.val + sv + c * 8);
    } else {
      a.kc[dk + c] = a.key[sk + c * a.ks_d];
      a.vc[dv + c] = a.val[sv + c * a.vs_d];
    }
  }
}

hipError_t launch_kv_write(const KVWriteArgs& a, bool vec, hipStream_t s) {
  const int per_row = vec ? a.D / 8 : a.D;
  const int64_t total = (int64_t)a.num_seqs * a.hkv * per_row;
  int64_t blocks = (total + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 65536) blocks = 65536;
  if (vec)
    kv_write_kernel<true><<<(unsigned)blocks, 256, 0, s>>>(a);
  else
    kv_write_kernel<false><<<(unsigned)blocks, 256, 0, s>>>(a);
  return hipGetLastError();
}

// Prefill block copy: source block j (tokens j*bs .. j*bs+bs-1 of the prompt
// slice) goes to cache block ids[j]; rows past num_tokens are written as zeros.
// This is the pool content the reference leaves after _copy_prefill_kv,
// engine/kernels/paged_attention_integration.py:278-326 (zero padding :315-317,
// index_copy_ of whole blocks :322-326).
template <bool VEC>
__global__ __launch_bounds__(256) void prefill_copy_kernel(PrefillCopyArgs a) {
  const int per_row = VEC ? a.D / 8 : a.D;
  const int64_t per_block = (int64_t)a.bs * a.hkv * per_row;
  const int64_t total = (int64_t)a.num_ids * per_block;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int j = (int)(i / per_block);
    int64_t r = i - (int64_t)j * per_block;
    const int row = (int)(r / ((int64_t)a.hkv * per_row));
    r -= (int64_t)row * a.hkv * per_row;
    const int h = (int)(r / per_row);
    const int c = (int)(r - (int64_t)h * per_row);
    const int id = a.ids[j];
    if (id < 0 || id >= a.num_blocks) continue;
    const int t = j * a.bs + row;
    const int64_t dk = (int64_t)id * a.kc_sb + (int64_t)row * a.kc_st + (int64_t)h * a.kc_sh;
    const int64_t dv = (int64_t)id * a.vc_sb + (int64_t)row * a.vc_st + (int64_t)h * a.vc_sh;
    if constexpr (VEC) {
      uint4 kx = {0u, 0u, 0u, 0u}, vx = {0u, 0u, 0u, 0u};
      if (t < a.num_tokens) {
        kx = *reinterpret_cast<const uint4*>(a.key + (int64_t)t * a.ks_t + (int64_t)h * a.ks_h + c * 8);
        vx = *reinterpret_cast<const uint4*>(a.val + (int64_t)t * a.vs_t + (int64_t)h * a.vs_h + c * 8);
      }
      *reinterpret_cast<uint4*>(a.kc + dk + c * 8) = kx;
      *reinterpret_cast<uint4*>(a.vc + dv + c * 8) = vx;
    } else {
      uint16_t kx = 0, vx = 0;
      if (t < a.num_tokens) {
        kx = a.key[(int64_t)t * a.ks_t + (int64_t)h * a.ks_h + (int64_t)c * a.ks_d];
        vx = a.val[(int64_t)t * a.vs_t + (int64_t)h * a.vs_h + (int64_t)c * a.vs_d];
      }
      a.kc[dk + c] = kx;
      a.vc[dv + c] = vx;
    }
  }
}

hipError_t launch_prefill_copy(const PrefillCopyArgs& a, bool vec, hipStream_t s) {
  const int per_row = vec ? a.D / 8 : a.D;
  const int64_t total = (int64_t)a.num_ids * a.bs * a.hkv * per_row;
  int64_t blocks = (total + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 65536) blocks = 65536;
  if (vec)
    prefill_copy_kernel<true><<<(unsigned)blocks, 256, 0, s>>>(a);
  else
    prefill_copy_kernel<false><<<(unsigned)blocks, 256, 0, s>>>(a);
  return hipGetLastError();
}

}  // namespace pa
