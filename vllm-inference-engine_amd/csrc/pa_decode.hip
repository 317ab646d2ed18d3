// Paged decode attention kernels for gfx950 (MI355X).
//
// Work unit: one 64-lane wavefront per (split, kv head, sequence). A split is a
// run of 16-token tiles of one sequence. For each tile the wavefront
//   * loads K and V rows with 16-byte loads, lane l taking token row l%16 and
//     an 8-element slice of head_dim,
//   * forms S^T = K * Q^T for the whole GQA group with v_mfma_f32_16x16x32_f16
//     (rows = 16 tokens, columns = up to 16 query heads of the group), so every
//     K byte is loaded once for all g query heads,
//   * keeps an online softmax per query head in the exp2 domain,
//   * forms O^T += V^T * P^T with v_mfma_f32_16x16x16_f16, V^T read from an LDS
//     copy of the tile and P split into an fp16 high part and an fp16
//     remainder so that the probabilities keep ~22 significant bits.
// Sequences longer than one split write fp32 partial records (max, denominator,
// unnormalised accumulator) that merge_kernel combines by log-sum-exp.
//
// MFMA register layouts used (16x16 output, wave64):
//   A operand: lane l holds row l%16, k-group l/16;  B operand: column l%16,
//   k-group l/16;  C/D: lane l holds rows 4*(l/16)+r (r = 0..3), column l%16.
// With S^T the output lane l holds head l%16 for tokens 4*(l/16)+r, which is
// exactly the B-operand layout of P^T in the second product, so probabilities
// never cross lanes.
#include "pa_common.h"

namespace pa {

__device__ inline f16x8 zero8() { return f16x8{0, 0, 0, 0, 0, 0, 0, 0}; }

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <int BS>
__device__ inline void split_token(int t, int bs_rt, int& lb, int& off) {
  if constexpr (BS > 0) {
    lb = t / BS;
    off = t % BS;
  } else {
    lb = t / bs_rt;
    off = t % bs_rt;
  }
}

// ---------------------------------------------------------------------------
// Batched / single-sequence online-softmax decode with split-K.
// ---------------------------------------------------------------------------
template <int D, int NT, int BS>
__global__ __launch_bounds__(64) void decode_split_kernel(DecodeArgs a) {
  constexpr int NC = D / 32;  // 16x16x32 products per score tile
  constexpr int ND = D / 16;  // 16-wide head_dim chunks of the output
  constexpr int LS = D + 8;   // LDS row stride of the staged V tile (halves)
  __shared__ __attribute__((aligned(16))) f16 lds_v[NT * 16 * LS];
  __shared__ int lds_ids[kMaxIds];

  const int lane = threadIdx.x;
  const int row = lane & 15;
  const int grp = lane >> 4;
  const int split = blockIdx.x;
  const int h = blockIdx.y;
  const int b = blockIdx.z;
  const int bs = BS > 0 ? BS : a.bs;

  const int L = clamped_len(a, b);
  const int ntiles = (L + 15) >> 4;
  const int nsplit = num_splits_for(ntiles, a.split_tiles);
  if (split >= nsplit) return;
  const int t0 = split * a.split_tiles;
  const int t1 = min(ntiles, t0 + a.split_tiles);

  // Stage the physical ids of the logical blocks this split touches.
  const int blk0 = (t0 * 16) / bs;
  const int blk_end = min((t1 * 16 + bs - 1) / bs, (L + bs - 1) / bs);
  const int32_t* btrow = a.bt + (int64_t)b * a.bt_sb;
  for (int i = lane; i < blk_end - blk0; i += 64) {
    const int id = btrow[(int64_t)(blk0 + i) * a.bt_sk];
    lds_ids[i] = min(max(id, 0), a.num_blocks - 1);
  }
  __syncthreads();

  // Q^T operand: column = query head `row` of this kv head's group.
  f16x8 qf[NC];
  {
    const int gq = min(row, a.g - 1);
    const f16* qp = a.q + (int64_t)b * a.q_sb + (int64_t)(h * a.g + gq) * a.q_sh + grp * 8;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const f16x8 t = *reinterpret_cast<const f16x8*>(qp + 32 * c);
      qf[c] = row < a.g ? t : zero8();
    }
  }

  const int64_t kh = (int64_t)h * a.k_sh + grp * 8;
  const int64_t vh = (int64_t)h * a.v_sh + grp * 8;

  // Load tile ti's K and V rows for this lane (token row `row`). Rows past the
  // sequence end read the split's first token instead and are zeroed later.
  auto load_tile = [&](int ti, f16x8 (&kt)[NC], f16x8 (&vt)[NC]) {
    int t = ti * 16 + row;
    if (t >= L) t = t0 * 16;
    int lb, off;
    split_token<BS>(t, bs, lb, off);
    const int64_t id = lds_ids[lb - blk0];
    const f16* kp = a.k + id * a.k_sb + (int64_t)off * a.k_st + kh;
    const f16* vp = a.v + id * a.v_sb + (int64_t)off * a.v_st + vh;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      kt[c] = *reinterpret_cast<const f16x8*>(kp + 32 * c);
      vt[c] = *reinterpret_cast<const f16x8*>(vp + 32 * c);
    }
  };

  float m_run = kNegInf;  // running max of head `row` (exp2 domain)
  float l_run = 0.f;      // this lane's share of the denominator
  f32x4 acc[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute_chunk = [&](int ti0, f16x8 (&kb)[NT][NC], f16x8 (&vb)[NT][NC]) {
    float xs[NT][4];
    float mloc = kNegInf;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int ti = ti0 + nt;
      if (ti < t1) {
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NC; ++c)
          s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb[nt][c], qf[c], s, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tok = ti * 16 + grp * 4 + r;
          const float x = tok < L ? s[r] * a.scale_log2 : kNegInf;
          xs[nt][r] = x;
          mloc = fmaxf(mloc, x);
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) xs[nt][r] = kNegInf;
      }
    }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
    const float m_new = fmaxf(m_run, mloc);
    const float alpha = fast_exp2(m_run - m_new);
    l_run *= alpha;
#pragma unroll
    for (int i = 0; i < ND; ++i) acc[i] *= alpha;
    m_run = m_new;

    // Stage V rows (zero past the sequence end so 0 * garbage cannot be NaN).
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int ti = ti0 + nt;
      if (ti < t1) {
        const bool valid = ti * 16 + row < L;
#pragma unroll
        for (int c = 0; c < NC; ++c)
          *reinterpret_cast<f16x8*>(&lds_v[(nt * 16 + row) * LS + 32 * c + grp * 8]) =
              valid ? vb[nt][c] : zero8();
      }
    }
    __syncthreads();
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int ti = ti0 + nt;
      if (ti < t1) {
        f16x4 ph, pl;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pr = fast_exp2(xs[nt][r] - m_run);
          l_run += pr;
          const f16 hi = (f16)pr;
          ph[r] = hi;
          pl[r] = (f16)(pr - (float)hi);
        }
#pragma unroll
        for (int nd = 0; nd < ND; ++nd) {
          f16x4 av;
#pragma unroll
          for (int r = 0; r < 4; ++r) av[r] = lds_v[(nt * 16 + grp * 4 + r) * LS + nd * 16 + row];
          acc[nd] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, ph, acc[nd], 0, 0, 0);
          acc[nd] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, pl, acc[nd], 0, 0, 0);
        }
      }
    }
    __syncthreads();
  };

  // Two register buffers: the next chunk's loads are in flight while the
  // current chunk is computed.
  f16x8 kb0[NT][NC], vb0[NT][NC], kb1[NT][NC], vb1[NT][NC];
  auto load_chunk = [&](int ti0, f16x8 (&kb)[NT][NC], f16x8 (&vb)[NT][NC]) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
      if (ti0 + nt < t1) load_tile(ti0 + nt, kb[nt], vb[nt]);
  };

  if (t0 < t1) load_chunk(t0, kb0, vb0);
  for (int ti = t0; ti < t1; ti += 2 * NT) {
    if (ti + NT < t1) load_chunk(ti + NT, kb1, vb1);
    compute_chunk(ti, kb0, vb0);
    if (ti + NT >= t1) break;
    if (ti + 2 * NT < t1) load_chunk(ti + 2 * NT, kb0, vb0);
    compute_chunk(ti + NT, kb1, vb1);
  }

  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);

  if (row >= a.g) return;
  if (nsplit == 1) {
    const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
    f16* op = a.out + (int64_t)b * a.o_sb + (int64_t)(h * a.g + row) * a.o_sh + grp * 4;
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) {
      f16x4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = (f16)(acc[nd][r] * inv);
      *reinterpret_cast<f16x4*>(op + nd * 16) = o;
    }
  } else {
    constexpr int REC = record_floats(D);
    float* rec = a.ws + (((int64_t)b * a.hkv + h) * a.max_splits + split) * REC;
    if (grp == 0) {
      rec[row] = m_run;
      rec[16 + row] = l_run;
    }
    float* ap = rec + 32 + row * D + grp * 4;
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) *reinterpret_cast<f32x4*>(ap + nd * 16) = acc[nd];
  }
}

// Log-sum-exp merge of the split-K partial records of one (sequence, kv head).
template <int D>
__global__ __launch_bounds__(256) void merge_kernel(DecodeArgs a) {
  constexpr int REC = record_floats(D);
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int L = clamped_len(a, b);
  const int nsplit = num_splits_for((L + 15) >> 4, a.split_tiles);
  if (nsplit <= 1) return;
  const float* recs = a.ws + ((int64_t)b * a.hkv + h) * a.max_splits * REC;
  for (int idx = threadIdx.x; idx < a.g * D; idx += blockDim.x) {
    const int hd = idx / D;
    const int d = idx - hd * D;
    float M = kNegInf;
    for (int s = 0; s < nsplit; ++s) M = fmaxf(M, recs[s * REC + hd]);
    float num = 0.f, den = 0.f;
    for (int s = 0; s < nsplit; ++s) {
      const float* r = recs + s * REC;
      const float w = fast_exp2(r[hd] - M);
      den += w * r[16 + hd];
      num += w * r[32 + hd * D + d];
    }
    a.out[(int64_t)b * a.o_sb + (int64_t)(h * a.g + hd) * a.o_sh + d] = (f16)(num / den);
  }
}

// ---------------------------------------------------------------------------
// Single-sequence two-pass decode (one 4-wave workgroup per kv head).
// Pass 1 writes the exp2-domain scores of every token to the workspace and
// reduces their maximum; a second pass sums exp2(score - max) into the
// denominator; pass 2 weights V by the normalised probabilities.
// ---------------------------------------------------------------------------
template <int D, int BS>
__global__ __launch_bounds__(256) void decode_v1_kernel(DecodeArgs a) {
  constexpr int NC = D / 32;
  constexpr int ND = D / 16;
  constexpr int LS = D + 8;
  __shared__ __attribute__((aligned(16))) f16 lds_v[4 * 16 * LS];
  __shared__ float red[4][16];
  __shared__ float head_m[16];
  __shared__ float head_den[16];
  __shared__ __attribute__((aligned(16))) float accred[16 * D];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int row = lane & 15;
  const int grp = lane >> 4;
  const int h = blockIdx.x;
  const int bs = BS > 0 ? BS : a.bs;
  const int L = clamped_len(a, 0);
  const int ntiles = (L + 15) >> 4;
  float* sc = a.ws + (int64_t)h * 16 * a.lpad;

  f16x8 qf[NC];
  {
    const int gq = min(row, a.g - 1);
    const f16* qp = a.q + (int64_t)(h * a.g + gq) * a.q_sh + grp * 8;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const f16x8 t = *reinterpret_cast<const f16x8*>(qp + 32 * c);
      qf[c] = row < a.g ? t : zero8();
    }
  }

  auto row_ptr = [&](int ti, const f16* base, int64_t sb, int64_t st, int64_t sh) {
    int t = ti * 16 + row;
    if (t >= L) t = 0;
    int lb, off;
    split_token<BS>(t, bs, lb, off);
    int id = a.bt[(int64_t)lb * a.bt_sk];
    id = min(max(id, 0), a.num_blocks - 1);
    return base + (int64_t)id * sb + (int64_t)off * st + (int64_t)h * sh + grp * 8;
  };

  // Pass 1: scores and their maximum.
  float mloc = kNegInf;
  for (int base = 0; base < ntiles; base += 4) {
    const int ti = base + wave;
    if (ti < ntiles) {
      const f16* kp = row_ptr(ti, a.k, a.k_sb, a.k_st, a.k_sh);
      f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c)
        s = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const f16x8*>(kp + 32 * c),
                                                   qf[c], s, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tok = ti * 16 + grp * 4 + r;
        const float x = tok < L ? s[r] * a.scale_log2 : kNegInf;
        sc[row * a.lpad + tok] = x;
        mloc = fmaxf(mloc, x);
      }
    }
  }
  mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
  mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
  if (grp == 0) red[wave][row] = mloc;
  __syncthreads();
  if (threadIdx.x < 16) {
    const int t = threadIdx.x;
    head_m[t] = fmaxf(fmaxf(red[0][t], red[1][t]), fmaxf(red[2][t], red[3][t]));
  }
  __syncthreads();

  // Denominator pass: 16 threads per head walk the stored scores.
  {
    const int hd = threadIdx.x >> 4;
    const int part = threadIdx.x & 15;
    const float mh = head_m[hd];
    float dsum = 0.f;
    for (int tok = part; tok < L; tok += 16) dsum += fast_exp2(sc[hd * a.lpad + tok] - mh);
    dsum += __shfl_xor(dsum, 1);
    dsum += __shfl_xor(dsum, 2);
    dsum += __shfl_xor(dsum, 4);
    dsum += __shfl_xor(dsum, 8);
    if (part == 0) head_den[hd] = dsum;
  }
  __syncthreads();

  // Pass 2: normalised probabilities times V.
  const float mh = head_m[row];
  const float inv_den = head_den[row] > 0.f ? 1.f / head_den[row] : 0.f;
  f32x4 acc[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  f16* my_v = lds_v + wave * 16 * LS;
  for (int base = 0; base < ntiles; base += 4) {
    const int ti = base + wave;
    const bool tv = ti < ntiles;
    if (tv) {
      const f16* vp = row_ptr(ti, a.v, a.v_sb, a.v_st, a.v_sh);
      const bool valid = ti * 16 + row < L;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const f16x8 vv = *reinterpret_cast<const f16x8*>(vp + 32 * c);
        *reinterpret_cast<f16x8*>(&my_v[row * LS + 32 * c + grp * 8]) = valid ? vv : zero8();
      }
    }
    __syncthreads();
    if (tv) {
      f16x4 ph, pl;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tok = ti * 16 + grp * 4 + r;
        const float pr = fast_exp2(sc[row * a.lpad + tok] - mh) * inv_den;
        const f16 hi = (f16)pr;
        ph[r] = hi;
        pl[r] = (f16)(pr - (float)hi);
      }
#pragma unroll
      for (int nd = 0; nd < ND; ++nd) {
        f16x4 av;
#pragma unroll
        for (int r = 0; r < 4; ++r) av[r] = my_v[(grp * 4 + r) * LS + nd * 16 + row];
        acc[nd] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, ph, acc[nd], 0, 0, 0);
        acc[nd] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, pl, acc[nd], 0, 0, 0);
      }
    }
    __syncthreads();
  }

  // Sum the four wavefronts' accumulators: waves 1..3 add into LDS in turn.
  for (int w = 1; w < 4; ++w) {
    if (wave == w) {
#pragma unroll
      for (int nd = 0; nd < ND; ++nd) {
        float* p = &accred[row * D + nd * 16 + grp * 4];
        f32x4 cur = w == 1 ? f32x4{0.f, 0.f, 0.f, 0.f} : *reinterpret_cast<f32x4*>(p);
        *reinterpret_cast<f32x4*>(p) = cur + acc[nd];
      }
    }
    __syncthreads();
  }
  if (wave == 0 && row < a.g) {
    f16* op = a.out + (int64_t)(h * a.g + row) * a.o_sh + grp * 4;
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) {
      const f32x4 tot = acc[nd] + *reinterpret_cast<const f32x4*>(&accred[row * D + nd * 16 + grp * 4]);
      f16x4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = (f16)tot[r];
      *reinterpret_cast<f16x4*>(op + nd * 16) = o;
    }
  }
}

// ---------------------------------------------------------------------------
// Host-side launchers (called from the C ABI after argument checks).
// ---------------------------------------------------------------------------
template <int D>
constexpr int chunk_tiles() {
  return D <= 64 ? 4 : (D <= 128 ? 2 : 1);
}

template <int D, int BS>
static hipError_t launch_split_bs(const DecodeArgs& a, int num_seqs, hipStream_t s) {
  dim3 grid(a.max_splits, a.hkv, num_seqs);
  decode_split_kernel<D, chunk_tiles<D>(), BS><<<grid, 64, 0, s>>>(a);
  if (a.max_splits > 1) merge_kernel<D><<<dim3(a.hkv, num_seqs), 256, 0, s>>>(a);
  return hipGetLastError();
}

template <int D>
static hipError_t launch_split_d(const DecodeArgs& a, int num_seqs, hipStream_t s) {
  switch (a.bs) {
    case 8: return launch_split_bs<D, 8>(a, num_seqs, s);
    case 16: return launch_split_bs<D, 16>(a, num_seqs, s);
    case 32: return launch_split_bs<D, 32>(a, num_seqs, s);
    default: return launch_split_bs<D, 0>(a, num_seqs, s);
  }
}

hipError_t launch_decode_split(const DecodeArgs& a, int D, int num_seqs, hipStream_t s) {
  switch (D) {
    case 32: return launch_split_d<32>(a, num_seqs, s);
    case 64: return launch_split_d<64>(a, num_seqs, s);
    case 128: return launch_split_d<128>(a, num_seqs, s);
    case 256: return launch_split_d<256>(a, num_seqs, s);
    default: return hipErrorInvalidValue;
  }
}

template <int D, int BS>
static hipError_t launch_v1_bs(const DecodeArgs& a, hipStream_t s) {
  decode_v1_kernel<D, BS><<<a.hkv, 256, 0, s>>>(a);
  return hipGetLastError();
}

template <int D>
static hipError_t launch_v1_d(const DecodeArgs& a, hipStream_t s) {
  switch (a.bs) {
    case 8: return launch_v1_bs<D, 8>(a, s);
    case 16: return launch_v1_bs<D, 16>(a, s);
    case 32: return launch_v1_bs<D, 32>(a, s);
    default: return launch_v1_bs<D, 0>(a, s);
  }
}

hipError_t launch_decode_v1(const DecodeArgs& a, int D, hipStream_t s) {
  switch (D) {
    case 32: return launch_v1_d<32>(a, s);
    case 64: return launch_v1_d<64>(a, s);
    case 128: return launch_v1_d<128>(a, s);
    case 256: return launch_v1_d<256>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace pa
