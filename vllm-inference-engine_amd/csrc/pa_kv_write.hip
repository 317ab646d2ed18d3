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
  kv_write_rows<VEC>(a, (int64_t)blockIdx.x * blockDim.x + threadIdx.x,
                     (int64_t)gridDim.x * blockDim.x);
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


// Fused rotary embedding + K/V write of one decode step.
//
// Replaces, per layer, transformers' apply_rotary_pos_emb on the new token's q
// and k (called at engine/kernels/paged_attention_integration.py:108-109)
// followed by the K/V write loop (:148-161). The rotation is the one
// transformers computes in fp16, op by op:
//   x_rot[j]       = fp16( fp16(x[j] * cos[j])             + fp16(-x[j + D/2] * sin[j]) )
//   x_rot[j + D/2] = fp16( fp16(x[j + D/2] * cos[j + D/2]) + fp16( x[j]       * sin[j + D/2]) )
// Each fp16 product and sum here is correctly rounded, which is what PyTorch's
// fp16 ops produce (they compute in fp32 and round once: an fp16 x fp16
// product is exact in fp32, and rounding an fp32 sum of two fp16 values to
// fp16 equals rounding the exact sum, since 24 >= 2 * 11 + 2). Queries go to
// q_out; keys and values go to the slot of position L-1 like kv_write_kernel.
// One thread handles 8 pairs (j, j + D/2) of one row when every row has unit
// stride and 16-byte alignment (VEC), one pair otherwise.
template <bool VEC>
__global__ __launch_bounds__(256) void rope_kv_write_kernel(RopeKVArgs a) {
  // Every product and sum is rounded on its own, as transformers' separate
  // fp16 ops round them: no contraction of x * c + y into a fused multiply-add.
#pragma clang fp contract(off)
  typedef _Float16 h16;
  const int half = a.D / 2;
  const int per_row = VEC ? half / 8 : half;
  const int rows = a.hq + 2 * a.hkv;  // q heads, then k heads, then v heads
  const int64_t total = (int64_t)a.num_seqs * rows * per_row;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(i % per_row);
    const int64_t r = i / per_row;
    const int row = (int)(r % rows);
    const int b = (int)(r / rows);
    const int j0 = VEC ? c * 8 : c;  // first pair index handled here
    // Destination: q_out for query rows, the cache slot for key / value rows.
    uint16_t* dst;
    const uint16_t* src;
    int64_t sd;
    bool rotate = true;
    if (row < a.hq) {
      src = a.q + (int64_t)b * a.qs_b + (int64_t)row * a.qs_h;
      sd = a.qs_d;
      dst = a.q_out + (int64_t)b * a.qo_b + (int64_t)row * a.qo_h;
    } else {
      const int L = a.lens ? a.lens[b] : a.uniform_len;
      if (L <= 0) continue;
      const int pos = L - 1;
      const int lb = pos / a.bs;
      if (lb >= a.max_blocks) continue;
      const int id = a.bt[(int64_t)b * a.bt_sb + (int64_t)lb * a.bt_sk];
      if (id < 0 || id >= a.num_blocks) continue;
      const int off = pos - lb * a.bs;
      if (row < a.hq + a.hkv) {
        const int h = row - a.hq;
        src = a.key + (int64_t)b * a.ks_b + (int64_t)h * a.ks_h;
        sd = a.ks_d;
        dst = a.kc + (int64_t)id * a.kc_sb + (int64_t)off * a.kc_st + (int64_t)h * a.kc_sh;
      } else {
        const int h = row - a.hq - a.hkv;
        src = a.val + (int64_t)b * a.vs_b + (int64_t)h * a.vs_h;
        sd = a.vs_d;
        dst = a.vc + (int64_t)id * a.vc_sb + (int64_t)off * a.vc_st + (int64_t)h * a.vc_sh;
        rotate = false;
      }
    }
    const uint16_t* cp = a.cos + (int64_t)b * a.cs_b;
    const uint16_t* sp = a.sin + (int64_t)b * a.ss_b;
    if constexpr (VEC) {
      uint4 lo = *reinterpret_cast<const uint4*>(src + j0);
      uint4 hi = *reinterpret_cast<const uint4*>(src + j0 + half);
      if (rotate) {
        const uint4 clo = *reinterpret_cast<const uint4*>(cp + j0);
        const uint4 chi = *reinterpret_cast<const uint4*>(cp + j0 + half);
        const uint4 slo = *reinterpret_cast<const uint4*>(sp + j0);
        const uint4 shi = *reinterpret_cast<const uint4*>(sp + j0 + half);
        const h16* x1 = reinterpret_cast<const h16*>(&lo);
        const h16* x2 = reinterpret_cast<const h16*>(&hi);
        const h16* c1 = reinterpret_cast<const h16*>(&clo);
        const h16* c2 = reinterpret_cast<const h16*>(&chi);
        const h16* s1 = reinterpret_cast<const h16*>(&slo);
        const h16* s2 = reinterpret_cast<const h16*>(&shi);
        uint4 olo, ohi;
        h16* o1 = reinterpret_cast<h16*>(&olo);
        h16* o2 = reinterpret_cast<h16*>(&ohi);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const h16 a1 = x1[e] * c1[e];
          const h16 b1 = -(x2[e] * s1[e]);
          o1[e] = a1 + b1;
          const h16 a2 = x2[e] * c2[e];
          const h16 b2 = x1[e] * s2[e];
          o2[e] = a2 + b2;
        }
        lo = olo;
        hi = ohi;
      }
      *reinterpret_cast<uint4*>(dst + j0) = lo;
      *reinterpret_cast<uint4*>(dst + j0 + half) = hi;
    } else {
      uint16_t lo = src[(int64_t)j0 * sd];
      uint16_t hi = src[(int64_t)(j0 + half) * sd];
      if (rotate) {
        const h16 x1 = __builtin_bit_cast(h16, lo), x2 = __builtin_bit_cast(h16, hi);
        const h16 c1 = __builtin_bit_cast(h16, cp[(int64_t)j0 * a.cs_d]);
        const h16 c2 = __builtin_bit_cast(h16, cp[(int64_t)(j0 + half) * a.cs_d]);
        const h16 s1 = __builtin_bit_cast(h16, sp[(int64_t)j0 * a.ss_d]);
        const h16 s2 = __builtin_bit_cast(h16, sp[(int64_t)(j0 + half) * a.ss_d]);
        const h16 a1 = x1 * c1;
        const h16 b1 = -(x2 * s1);
        const h16 a2 = x2 * c2;
        const h16 b2 = x1 * s2;
        lo = __builtin_bit_cast(uint16_t, (h16)(a1 + b1));
        hi = __builtin_bit_cast(uint16_t, (h16)(a2 + b2));
      }
      dst[j0] = lo;  // q_out and the caches have unit head_dim stride
      dst[j0 + half] = hi;
    }
  }
}

hipError_t launch_rope_kv_write(const RopeKVArgs& a, bool vec, hipStream_t s) {
  const int per_row = vec ? a.D / 16 : a.D / 2;
  const int64_t total = (int64_t)a.num_seqs * (a.hq + 2 * a.hkv) * per_row;
  int64_t blocks = (total + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 65536) blocks = 65536;
  if (vec)
    rope_kv_write_kernel<true><<<(unsigned)blocks, 256, 0, s>>>(a);
  else
    rope_kv_write_kernel<false><<<(unsigned)blocks, 256, 0, s>>>(a);
  return hipGetLastError();
}

}  // namespace pa
