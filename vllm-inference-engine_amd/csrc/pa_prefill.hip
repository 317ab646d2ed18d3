// Paged prefill attention for gfx950 (MI355X): the new tokens of each sequence
// (a prompt suffix after cached prefix blocks, or a whole prompt) attend
// causally over the sequence's pool rows -- the cached prefix plus their own
// K/V, which are written to the pool before this kernel runs. New token i of a
// sequence with context length L and n new tokens sits at position L - n + i
// and sees pool rows 0 .. L - n + i.
//
// Work split. The (token, query head) pairs of one sequence and one kv head
// form a list of n * g columns, token-major. A workgroup of four wavefronts
// takes 64 consecutive columns (16 per wavefront), so the K/V rows it stages
// serve all g query heads of the kv head at once. Workgroups with the latest
// columns see the most keys; they are numbered first so the longest run
// starts first.
//
// Per 64-key tile the workgroup loads K and V rows (16-byte loads, block id
// per row from the table) into LDS, one tile ahead in registers. Each
// wavefront computes S^T = K Q^T on MFMA (16 keys x 16 columns per
// instruction, K read in the operand layout, Q kept in registers), masks keys
// past each column's position, updates its online softmax in the exp2 domain
// and accumulates O^T += V^T P^T on MFMA with V^T read transposed from LDS --
// the operand layouts of the decode kernel, with columns that are (token,
// head) pairs instead of the heads of one token.
#include "pa_tiles.h"

namespace pa {

using namespace tiles;

template <int D>
__global__ __launch_bounds__(256) void prefill_attn_kernel(PrefillAttnArgs a) {
  constexpr int NW = 4;
  constexpr int COLS = 16 * NW;  // columns per workgroup
  constexpr int KT = 64;         // keys per staged tile
  constexpr int NS = KT / 16;    // 16-key sub-tiles per tile
  constexpr int NC = D / 32;
  constexpr int ND = D / 16;
  constexpr int LS = D + 8;      // LDS row stride in halves
  constexpr int CPR = D / 8;     // 16-byte pieces per key row of one head
  constexpr int PER = KT * CPR / (64 * NW);
  static_assert(PER * 64 * NW == KT * CPR, "a tile must split evenly over the workgroup");

  __shared__ __attribute__((aligned(16))) f16 ks[KT * LS];
  __shared__ __attribute__((aligned(16))) f16 vs[KT * LS];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int row = lane & 15;
  const int grp = lane >> 4;

  const int per_cb = a.num_seqs * a.hkv;
  const int cb = a.col_blocks - 1 - (int)(blockIdx.x / per_cb);
  const int rest = (int)(blockIdx.x % per_cb);
  const int b = rest / a.hkv;
  const int h = rest - b * a.hkv;

  int q0 = a.qstart[b];
  int q1 = a.qstart[b + 1];
  q0 = min(max(q0, 0), a.num_tokens);
  q1 = min(max(q1, q0), a.num_tokens);
  const int qlen = q1 - q0;
  const int ncols = qlen * a.g;
  const int cfirst = cb * COLS;
  if (cfirst >= ncols) return;
  const int clast = min(cfirst + COLS, ncols) - 1;
  const int cap = a.max_blocks * a.bs;
  int L = a.lens[b];
  L = L < 0 ? 0 : (L > cap ? cap : L);
  const int pos0 = L - qlen;                  // position of the first new token
  const int kmax = pos0 + clast / a.g + 1;    // keys [0, kmax) are read
  const int pmin = pos0 + cfirst / a.g;       // every column sees keys [0, pmin]

  // This lane's column; columns past the list compute as the last valid one
  // and are not stored.
  const int col = cfirst + wave * 16 + row;
  const bool col_ok = col < ncols;
  const int cc = col_ok ? col : clast;
  const int t = cc / a.g;
  const int j = cc - t * a.g;
  const int pos = pos0 + t;
  f16* op = a.out + (int64_t)(q0 + t) * a.o_st + (int64_t)(h * a.g + j) * a.o_sh + grp * 4;

  if (kmax <= 0) {  // context shorter than the new tokens: no key is visible to any column
    if (col_ok) {
#pragma unroll
      for (int nd = 0; nd < ND; ++nd) *reinterpret_cast<f16x4*>(op + nd * 16) = f16x4{0, 0, 0, 0};
    }
    return;
  }
  const int pos_c = pos < 0 ? 0 : pos;  // such columns are written as zeros below

  f16x8 qf[NC];
  {
    const f16* qp = a.q + (int64_t)(q0 + t) * a.q_st + (int64_t)(h * a.g + j) * a.q_sh + grp * 8;
#pragma unroll
    for (int c = 0; c < NC; ++c) qf[c] = *reinterpret_cast<const f16x8*>(qp + 32 * c);
  }

  const int32_t* btrow = a.bt + (int64_t)b * a.bt_sb;
  const f16* kbase = a.k + (int64_t)h * a.k_sh;
  const f16* vbase = a.v + (int64_t)h * a.v_sh;
  u32x4 kr[PER], vr[PER];
  // Piece f = 256 i + tid of a tile is key row f / CPR, halves (f % CPR) * 8.
  auto fetch = [&](int kt) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int f = i * 64 * NW + tid;
      const int r = f / CPR;
      const int c8 = (f % CPR) * 8;
      const int key = kt * KT + r;
      if (key < kmax) {
        int id = btrow[(int64_t)(key / a.bs) * a.bt_sk];
        id = min(max(id, 0), a.num_blocks - 1);
        const int64_t off = key % a.bs;
        kr[i] = *reinterpret_cast<const u32x4*>(kbase + id * a.k_sb + off * a.k_st + c8);
        vr[i] = *reinterpret_cast<const u32x4*>(vbase + id * a.v_sb + off * a.v_st + c8);
      } else {
        // Rows past the last key are zeros: masked scores give p = 0, and
        // 0 * (zero row) never makes a NaN.
        kr[i] = u32x4{0u, 0u, 0u, 0u};
        vr[i] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int f = i * 64 * NW + tid;
      const int r = f / CPR;
      const int c8 = (f % CPR) * 8;
      *reinterpret_cast<u32x4*>(&ks[r * LS + c8]) = kr[i];
      *reinterpret_cast<u32x4*>(&vs[r * LS + c8]) = vr[i];
    }
  };

  float m_run = kNegInf, l_run = 0.f;
  f32x4 acc[ND];
#pragma unroll
  for (int nd = 0; nd < ND; ++nd) acc[nd] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int ntiles = (kmax + KT - 1) / KT;
  fetch(0);
  for (int kt = 0; kt < ntiles; ++kt) {
    __syncthreads();  // every wavefront is done reading the previous tile
    stash();
    __syncthreads();
    if (kt + 1 < ntiles) fetch(kt + 1);

    // Scores of the tile: lane (row, grp) holds keys 16 s + 4 grp + r of column `row`.
    float xs[NS][4];
    float mloc = kNegInf;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int kb = kt * KT + s * 16;
      if (kb < kmax) {  // workgroup-uniform
        const f16* kp = ks + (s * 16 + row) * LS + grp * 8;
        f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NC; ++c)
          sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const f16x8*>(kp + 32 * c),
                                                      qf[c], sc, 0, 0, 0);
        if (kb + 15 <= pmin) {  // every column sees the whole sub-tile
#pragma unroll
          for (int r = 0; r < 4; ++r) xs[s][r] = sc[r] * a.scale_log2;
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            xs[s][r] = kb + grp * 4 + r <= pos_c ? sc[r] * a.scale_log2 : kNegInf;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) mloc = fmaxf(mloc, xs[s][r]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) xs[s][r] = kNegInf;
      }
    }
    // Key 0 is in the first tile and visible to every column, so m_run is
    // finite from the first tile on and no exp2 sees -inf - -inf.
    mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
    const float m_new = fmaxf(m_run, mloc);
    const float alpha = fast_exp2(m_run - m_new);
    l_run *= alpha;
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) acc[nd] *= alpha;
    m_run = m_new;

#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int kb = kt * KT + s * 16;
      if (kb < kmax) {
        // P^T as the B operand: the score layout already is (column `row`,
        // keys 4 grp + r). fp16 high part plus fp16 remainder keeps ~22 bits.
        f16x4 ph, pl;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pr = fast_exp2(xs[s][r] - m_run);
          l_run += pr;
          const f16 hi = (f16)pr;
          ph[r] = hi;
          pl[r] = (f16)(pr - (float)hi);
        }
        // V^T operand: lane (row, grp) needs V[4 grp + r][16 nd + row], r = 0..3,
        // which one transposing read of key rows 4 grp .. 4 grp + 3 delivers.
        const f16* vt = vs + (s * 16 + grp * 4 + (row >> 2)) * LS + (row & 3) * 4;
#pragma unroll
        for (int nd = 0; nd < ND; ++nd) {
          const f16x4 av = lds_read_tr16(vt + nd * 16);
          acc[nd] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, ph, acc[nd], 0, 0, 0);
          acc[nd] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, pl, acc[nd], 0, 0, 0);
        }
      }
    }
  }

  // Denominator: each lane summed its own four keys per sub-tile.
  float l = l_run;
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  if (col_ok) {
    const float inv = pos >= 0 ? 1.f / l : 0.f;
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) {
      f16x4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = (f16)(acc[nd][r] * inv);
      *reinterpret_cast<f16x4*>(op + nd * 16) = o;
    }
  }
}

template <int D>
static hipError_t launch_prefill_d(const PrefillAttnArgs& a, hipStream_t s) {
  const int64_t grid = (int64_t)a.col_blocks * a.num_seqs * a.hkv;
  hipLaunchKernelGGL(prefill_attn_kernel<D>, dim3((unsigned)grid), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_prefill_attn(const PrefillAttnArgs& a, int D, hipStream_t s) {
  switch (D) {
    case 32: return launch_prefill_d<32>(a, s);
    case 64: return launch_prefill_d<64>(a, s);
    case 128: return launch_prefill_d<128>(a, s);
    case 256: return launch_prefill_d<256>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace pa
