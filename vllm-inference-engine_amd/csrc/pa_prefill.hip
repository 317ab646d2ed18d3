// Paged prefill attention for gfx950 (MI355X): the new tokens of each sequence
// (a prompt suffix after cached prefix blocks, or a whole prompt) attend
// causally over the sequence's pool rows -- the cached prefix plus their own
// K/V, which are written to the pool before this kernel runs. New token i of a
// sequence with context length L and n new tokens sits at position L - n + i
// and sees pool rows 0 .. L - n + i.
//
// Work split. The (token, query head) pairs of one sequence and one kv head
// form a list of n * g columns, token-major. A workgroup takes 128
// consecutive columns (four wavefronts of two groups of 16 columns, where each
// K or V operand read from LDS feeds two MFMAs, or up to head_dim 64 eight
// wavefronts of one group; 64 columns, one group per wavefront, at head_dim
// 256), so the K/V rows it stages serve all g query heads of the kv head at
// once. Workgroups with the latest columns see the most keys; they
// are numbered first so the longest runs start first.
//
// Per key tile (128 keys up to head_dim 64, else 64) the workgroup loads K
// and V rows (16-byte loads, block id per row from the table, fetched a tile
// earlier) into registers one tile ahead, and stores them into two LDS
// buffers used alternately, one barrier per tile. Each wavefront computes
// S^T = K Q^T on MFMA (16 keys x 16 columns per instruction, K read in the
// operand layout, Q kept in registers), masks keys past each column's
// position (only on tiles that cross one), keeps an online softmax in the
// exp2 domain whose maximum is raised lazily, and accumulates O^T += V^T P^T
// with fp16 probabilities on K=32 MFMAs, V^T read transposed from LDS -- the
// operand layouts of the decode kernel, with columns that are (token, head)
// pairs instead of the heads of one token.
#include "pa_tiles.h"

namespace pa {

using namespace tiles;

template <int D, int BS, int CG, int NW>
__global__ __launch_bounds__(64 * NW) void prefill_attn_kernel(PrefillAttnArgs a) {
  constexpr int COLS = 16 * CG * NW;  // columns per workgroup
  constexpr int KT = prefill_key_tile(D);  // keys per staged tile
  constexpr int NS = KT / 16;         // 16-key sub-tiles per tile
  constexpr int NC = D / 32;
  constexpr int ND = D / 16;
  constexpr int LS = D + 8;           // LDS row stride in halves
  constexpr int CPR = D / 8;          // 16-byte pieces per key row of one head
  constexpr int PER = KT * CPR / (64 * NW);
  constexpr int BUF = KT * LS;        // halves of one staged K (or V) tile
  static_assert(PER * 64 * NW == KT * CPR, "a tile must split evenly over the workgroup");
  static_assert(NS % 2 == 0, "sub-tiles are paired for the P V products");

  __shared__ __attribute__((aligned(16))) f16 ks[2 * BUF];
  __shared__ __attribute__((aligned(16))) f16 vs[2 * BUF];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int row = lane & 15;
  const int grp = lane >> 4;

  // Workgroup -> (column block, key split, sequence, kv head); the column
  // blocks with the most keys come first.
  const int per_cb = a.num_seqs * a.hkv;
  const int cbi = (int)(blockIdx.x / (per_cb * a.max_splits));
  const int rem = (int)(blockIdx.x - (unsigned)cbi * per_cb * a.max_splits);
  const int split = rem / per_cb;
  const int rest = rem - split * per_cb;
  const int cb = a.col_blocks - 1 - cbi;
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
  const int pos0 = L - qlen;                // position of the first new token
  const int kmax = pos0 + clast / a.g + 1;  // keys [0, kmax) are read
  const int pmin = pos0 + cfirst / a.g;     // every column sees keys [0, pmin]
  const int ntiles = kmax > 0 ? (kmax + KT - 1) / KT : 0;
  const int nsplit = ntiles > a.split_tiles ? (ntiles + a.split_tiles - 1) / a.split_tiles : 1;
  if (split >= nsplit) return;
  const int t0 = split * a.split_tiles;                       // this workgroup's key tiles
  const int t1 = min(t0 + a.split_tiles, ntiles);             // [t0, t1)

  // This lane's columns (one per column group); columns past the list compute
  // as the last valid one and are not stored.
  bool col_ok[CG];
  int pos[CG], pos_c[CG];
  f16* op[CG];
  f16x8 qf[CG][NC];
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    const int col = cfirst + (wave * CG + cg) * 16 + row;
    col_ok[cg] = col < ncols;
    const int cc = col_ok[cg] ? col : clast;
    const int t = cc / a.g;
    const int j = cc - t * a.g;
    pos[cg] = pos0 + t;
    pos_c[cg] = pos[cg] < 0 ? 0 : pos[cg];  // such columns are written as zeros below
    op[cg] = a.out + (int64_t)(q0 + t) * a.o_st + (int64_t)(h * a.g + j) * a.o_sh + grp * 4;
    const f16* qp = a.q + (int64_t)(q0 + t) * a.q_st + (int64_t)(h * a.g + j) * a.q_sh + grp * 8;
#pragma unroll
    for (int c = 0; c < NC; ++c) qf[cg][c] = *reinterpret_cast<const f16x8*>(qp + 32 * c);
  }

  if (kmax <= 0) {  // context shorter than the new tokens: no key is visible to any column
#pragma unroll
    for (int cg = 0; cg < CG; ++cg)
      if (col_ok[cg]) {
#pragma unroll
        for (int nd = 0; nd < ND; ++nd)
          *reinterpret_cast<f16x4*>(op[cg] + nd * 16) = f16x4{0, 0, 0, 0};
      }
    return;
  }

  const int32_t* btrow = a.bt + (int64_t)b * a.bt_sb;
  const f16* kbase = a.k + (int64_t)h * a.k_sh;
  const f16* vbase = a.v + (int64_t)h * a.v_sh;
  const int bs = BS > 0 ? BS : a.bs;
  u32x4 kr[PER], vr[PER];
  int ids[PER];
  // Piece f = 64 NW i + tid of a tile is key row f / CPR, halves (f % CPR) * 8.
  // The block ids of a tile are loaded one tile before its K/V, so a K/V load
  // never waits on the table read it depends on.
  // Element strides fit 32 bits (the host checks it): a block's offset is one
  // 32 x 32 -> 64-bit multiply-add, the row offset inside it 32-bit. This
  // address arithmetic runs for every 16-byte piece of every tile, so it is
  // kept to a few instructions.
  const uint32_t k_sb = (uint32_t)a.k_sb, v_sb = (uint32_t)a.v_sb;
  const uint32_t k_st = (uint32_t)a.k_st, v_st = (uint32_t)a.v_st;
  const uint32_t bt_sk = (uint32_t)a.bt_sk;
  // Rows past the last key are loaded from the last key's row instead
  // (clamped, so every load is a valid pool row and no branch splits the
  // loads): their scores fall past every column's position and are masked,
  // and p = 0 times a finite row adds nothing.
  //
  // Tiles wholly below kmax, when the block size divides the key tile: a
  // piece's row in the tile -- so its table column within the tile, its row in
  // the block and its 16-byte column -- is the same in every tile, and only
  // the block id changes. Its K and V addresses are then the block id times
  // the block stride plus a base fixed for the piece, and its block-id address
  // a fixed one plus a tile offset common to the workgroup: a few vector
  // instructions per piece instead of the general form's clamps, divisions
  // and two 64-bit multiply-adds per load.
  constexpr bool FIXED = BS > 0 && KT % BS == 0 && D <= 128;  // at head_dim 256 the bases cost occupancy
  const f16* kfix[PER];
  const f16* vfix[PER];
  const int32_t* idfix[PER];
  if constexpr (FIXED) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int f = i * 64 * NW + tid;
      const uint32_t r = (uint32_t)(f / CPR), c8 = (uint32_t)(f % CPR) * 8;
      kfix[i] = kbase + ((r % BS) * k_st + c8);
      vfix[i] = vbase + ((r % BS) * v_st + c8);
      idfix[i] = btrow + (r / BS) * bt_sk;
    }
  }
  auto whole = [&](int kt) { return FIXED && (kt + 1) * KT <= kmax; };  // workgroup-uniform
  auto fetch_ids = [&](int kt) {
    if (whole(kt)) {
      const uint32_t to = (uint32_t)kt * (uint32_t)(KT / (BS > 0 ? BS : 1)) * bt_sk;
#pragma unroll
      for (int i = 0; i < PER; ++i) ids[i] = idfix[i][to];
      return;
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int key = min(kt * KT + (i * 64 * NW + tid) / CPR, kmax - 1);
      ids[i] = btrow[(uint32_t)(key / bs) * bt_sk];
    }
  };
  auto fetch_kv = [&](int kt) {
    if (whole(kt)) {
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const uint32_t id = (uint32_t)min(max(ids[i], 0), a.num_blocks - 1);
        kr[i] = *reinterpret_cast<const u32x4*>(kfix[i] + (uint64_t)id * k_sb);
        vr[i] = *reinterpret_cast<const u32x4*>(vfix[i] + (uint64_t)id * v_sb);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int f = i * 64 * NW + tid;
      const uint32_t c8 = (f % CPR) * 8;
      const int key = min(kt * KT + f / CPR, kmax - 1);
      const uint32_t id = (uint32_t)min(max(ids[i], 0), a.num_blocks - 1);
      const uint32_t off = (uint32_t)(key % bs);
      kr[i] = *reinterpret_cast<const u32x4*>(kbase + (uint64_t)id * k_sb + (off * k_st + c8));
      vr[i] = *reinterpret_cast<const u32x4*>(vbase + (uint64_t)id * v_sb + (off * v_st + c8));
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int f = i * 64 * NW + tid;
      const int r = f / CPR;
      const int c8 = (f % CPR) * 8;
      *reinterpret_cast<u32x4*>(&ks[buf * BUF + r * LS + c8]) = kr[i];
      *reinterpret_cast<u32x4*>(&vs[buf * BUF + r * LS + c8]) = vr[i];
    }
  };

  float m_run[CG], l_run[CG];
  f32x4 acc[CG][ND];
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    m_run[cg] = kNegInf;
    l_run[cg] = 0.f;
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) acc[cg][nd] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // Two LDS buffers: tile kt is read from buffer kt % 2 while tile kt + 1 is
  // written to the other, so each tile needs one barrier.
  fetch_ids(t0);
  fetch_kv(t0);
  fetch_ids(t0 + 1);
  stash(t0 & 1);
  __syncthreads();
  // Every load issued so far (the query fragments included, which the
  // compiler may place after the first tile's loads) is complete before the
  // loop: otherwise the loop's wait counts must assume the query loads may
  // still be pending at its first products, and every tile's score products
  // would wait for the next tile's K/V loads issued just before them.
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_sched_barrier(0);
  for (int kt = t0; kt < t1; ++kt) {
    const bool more = kt + 1 < t1;
    if (more) {
      fetch_kv(kt + 1);
      fetch_ids(kt + 2);
    }
    const f16* kt_lds = ks + (kt & 1) * BUF;
    const f16* vt_lds = vs + (kt & 1) * BUF;

    // Raw scores of the whole tile, without branches: lane (row, grp) holds
    // keys 16 s + 4 grp + r of its column in each group. Rows past the last
    // key hold copies of the last key's row; the mask below removes them
    // with the causal cut.
    f32x4 sc[CG][NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      f16x8 kf[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c)
        kf[c] = *reinterpret_cast<const f16x8*>(kt_lds + (s * 16 + row) * LS + grp * 8 + 32 * c);
#pragma unroll
      for (int cg = 0; cg < CG; ++cg) {
        sc[cg][s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NC; ++c)
          sc[cg][s] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[c], qf[cg][c], sc[cg][s], 0, 0, 0);
      }
    }
    if (kt * KT + KT - 1 > pmin) {  // workgroup-uniform: a tile crossing some column's position
#pragma unroll
      for (int cg = 0; cg < CG; ++cg)
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (kt * KT + s * 16 + grp * 4 + r > pos_c[cg]) sc[cg][s][r] = kNegInf;
    }
    // Probabilities with the running maximum as it stands. The maxima are
    // taken only when that fails: for a column's first tile (its maximum is
    // still -inf) or when a score exceeds it by 16 or more, so that a
    // probability overflows fp16 -- which makes the fp16 denominator sum
    // infinite (or NaN). Probabilities thus stay below 2^16, and most tiles
    // skip the maxima and the accumulator rescale.
    f16x8 pb[NS / 2][CG];
    float lt[CG];
    auto probs = [&]() {
#pragma unroll
      for (int cg = 0; cg < CG; ++cg) {
        // A column with no visible key yet keeps m = -inf; any finite offset
        // then gives p = 0 for its -inf scores.
        const float nm = m_run[cg] == kNegInf ? 0.f : -m_run[cg];
        lt[cg] = 0.f;
#pragma unroll
        for (int sp = 0; sp < NS / 2; ++sp) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            pb[sp][cg][r] = (f16)fast_exp2(__builtin_fmaf(sc[cg][2 * sp][r], a.scale_log2, nm));
            pb[sp][cg][4 + r] =
                (f16)fast_exp2(__builtin_fmaf(sc[cg][2 * sp + 1][r], a.scale_log2, nm));
          }
#pragma unroll
          for (int i = 0; i < 4; ++i)
            lt[cg] = __builtin_amdgcn_fdot2(f16x2{pb[sp][cg][2 * i], pb[sp][cg][2 * i + 1]},
                                            f16x2{(f16)1.f, (f16)1.f}, lt[cg], false);
        }
      }
    };
    probs();
    bool redo = false;
#pragma unroll
    for (int cg = 0; cg < CG; ++cg)
      redo |= m_run[cg] == kNegInf ||
              (__builtin_bit_cast(uint32_t, lt[cg]) & 0x7f800000u) == 0x7f800000u;
    if (__builtin_amdgcn_ballot_w64(redo) != 0) {  // wavefront-uniform
      // Maxima in the exp2 domain (the scale is positive, so it commutes
      // with the maximum), raise, rescale, recompute.
#pragma unroll
      for (int cg = 0; cg < CG; ++cg) {
        float m = kNegInf;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          m = fmaxf(fmaxf(m, sc[cg][s][0]), sc[cg][s][1]);  // one v_max3_f32 each
          m = fmaxf(fmaxf(m, sc[cg][s][2]), sc[cg][s][3]);
        }
        m = fmaxf(m, __shfl_xor(m, 16));
        m = fmaxf(m, __shfl_xor(m, 32));
        const float m_new = fmaxf(m_run[cg], m * a.scale_log2);
        // A column with no visible key yet (only in a split after the first)
        // stays at -inf, and -inf - -inf would make its alpha NaN.
        const float alpha = m_new == kNegInf ? 1.f : fast_exp2(m_run[cg] - m_new);
        l_run[cg] *= alpha;
#pragma unroll
        for (int nd = 0; nd < ND; ++nd) acc[cg][nd] *= alpha;
        m_run[cg] = m_new;
      }
      probs();
    }
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) l_run[cg] += lt[cg];

    // O^T += V^T P^T over pairs of sub-tiles, 32 keys per MFMA: operand index
    // k = 8 grp + i stands for key 16 s0 + 4 grp + i (i < 4) or 16 s1 + 4 grp
    // + i - 4, in both the V^T and the P^T operand. Denominators sum the same
    // fp16-rounded probabilities the products use.
#pragma unroll
    for (int sp = 0; sp < NS / 2; ++sp) {
      // V^T operand: lane (row, grp) needs V[16 s + 4 grp + r][16 nd + row],
      // r = 0..3, which one transposing read of four key rows delivers.
      const f16* v0 = vt_lds + (2 * sp * 16 + grp * 4 + (row >> 2)) * LS + (row & 3) * 4;
      const f16* v1 = v0 + 16 * LS;
#pragma unroll
      for (int nd = 0; nd < ND; ++nd) {
        const f16x4 a0 = lds_read_tr16(v0 + nd * 16);
        const f16x4 a1 = lds_read_tr16(v1 + nd * 16);
        const f16x8 av = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
#pragma unroll
        for (int cg = 0; cg < CG; ++cg)
          acc[cg][nd] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, pb[sp][cg], acc[cg][nd], 0, 0, 0);
      }
    }

    if (more) stash((kt + 1) & 1);
    __syncthreads();
  }

  // Denominators: each lane summed its own keys.
  float lsum[CG];
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    float l = l_run[cg];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    lsum[cg] = l;
  }
  if (nsplit == 1) {
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) {
      if (col_ok[cg]) {
        const float inv = pos[cg] >= 0 ? 1.f / lsum[cg] : 0.f;
#pragma unroll
        for (int nd = 0; nd < ND; ++nd) {
          f16x4 o;
#pragma unroll
          for (int r = 0; r < 4; ++r) o[r] = (f16)(acc[cg][nd][r] * inv);
          *reinterpret_cast<f16x4*>(op[cg] + nd * 16) = o;
        }
      }
    }
    return;
  }

  // Several splits: leave this split's record -- per column the running
  // maximum, the denominator and the unnormalised accumulators -- with
  // device-coherent stores (the splits run on any XCD), then count the
  // arrival. The split completing the count merges every record in split
  // order and resets the counter for the next launch.
  constexpr int REC = COLS * (D + 2);  // floats of one record: maxima, denominators, accumulators
  const int64_t blk = ((int64_t)b * a.hkv + h) * a.col_blocks + cb;
  const auto rr = tile_rsrc(a.recs + blk * a.max_splits * REC, nsplit * REC * 4);
  {
    const int rb = split * REC * 4;  // byte offset of this split's record
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) {
      const int cl = (wave * CG + cg) * 16 + row;
      if (grp == 0) {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, m_run[cg]), rr,
                                              rb + cl * 4, 0, 16);
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, lsum[cg]), rr,
                                              rb + (COLS + cl) * 4, 0, 16);
      }
#pragma unroll
      for (int nd = 0; nd < ND; ++nd)
        store_coherent16(rr, rb + (2 * COLS + cl * D + nd * 16 + grp * 4) * 4, acc[cg][nd]);
    }
  }
  __shared__ int s_last;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0)
    s_last = __hip_atomic_fetch_add(a.cnt + blk, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             nsplit - 1;
  __syncthreads();
  if (!s_last) return;

  // Merge: TPC threads per column, each DPT consecutive values of head_dim,
  // read as 16-byte device-coherent loads. Records are combined MS at a time
  // (as many as registers allow) with a running maximum -- log-sum-exp in
  // split order -- so a merge costs about one memory round trip per MS splits.
  constexpr int TPC = 64 * NW / COLS;
  constexpr int DPT = D / TPC;
  constexpr int MS = DPT <= 32 ? 2 : 1;
  {
    const int cl = tid / TPC;
    const int d0 = (tid - cl * TPC) * DPT;
    const int col = cfirst + cl;
    if (col < ncols) {
      const int tt = col / a.g;
      const int jj = col - tt * a.g;
      f16* o = a.out + (int64_t)(q0 + tt) * a.o_st + (int64_t)(h * a.g + jj) * a.o_sh + d0;
      f32x4 v[DPT / 4];
#pragma unroll
      for (int i = 0; i < DPT / 4; ++i) v[i] = f32x4{0.f, 0.f, 0.f, 0.f};
      float L = 0.f;
      if (pos0 + tt >= 0) {
        float Mr = kNegInf;
        for (int sp = 0; sp < nsplit; sp += MS) {
          f32x4 pt[MS][DPT / 4];
          float m[MS], l[MS];
#pragma unroll
          for (int k = 0; k < MS; ++k) {
            const bool in = sp + k < nsplit;
            const int rb = (in ? sp + k : sp) * REC * 4;
#pragma unroll
            for (int i = 0; i < DPT / 4; ++i)
              pt[k][i] = load_coherent16(rr, rb + (2 * COLS + cl * D + d0 + 4 * i) * 4);
            m[k] = in ? load_coherent4(rr, rb + cl * 4) : kNegInf;
            l[k] = in ? load_coherent4(rr, rb + (COLS + cl) * 4) : 0.f;
          }
          // A split that saw no key of this column has m = -inf and l = 0.
          float mn = Mr;
#pragma unroll
          for (int k = 0; k < MS; ++k) mn = fmaxf(mn, m[k]);
          if (mn == kNegInf) continue;
          const float al = Mr == kNegInf ? 0.f : fast_exp2(Mr - mn);
          L *= al;
#pragma unroll
          for (int i = 0; i < DPT / 4; ++i) v[i] *= al;
#pragma unroll
          for (int k = 0; k < MS; ++k) {
            const float w = m[k] == kNegInf ? 0.f : fast_exp2(m[k] - mn);
            L += l[k] * w;
#pragma unroll
            for (int i = 0; i < DPT / 4; ++i) v[i] += w * pt[k][i];
          }
          Mr = mn;
        }
        L = 1.f / L;
      }
#pragma unroll
      for (int i = 0; i < DPT / 4; ++i) {
        f16x4 h4;
#pragma unroll
        for (int r = 0; r < 4; ++r) h4[r] = (f16)(v[i][r] * L);
        *reinterpret_cast<f16x4*>(o + 4 * i) = h4;
      }
    }
  }
  if (tid == 0) __hip_atomic_store(a.cnt + blk, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A column block of 64 CG columns runs as four wavefronts of CG groups of 16
// columns; up to head_dim 64, a block of two groups per wavefront may run as
// eight wavefronts of one group instead (a.wave_groups, chosen by the host):
// four wavefronts per SIMD instead of two (125 VGPRs instead of 230 at head_dim
// 64). Each column's arithmetic is the same except where a wavefront raises its
// running maxima: it does so for all the columns it holds at once (16 or 32),
// so the two forms agree to rounding and mostly bit for bit. At head_dim 128
// the eight-wavefront form would hold one workgroup per CU (148 VGPRs), so four
// wavefronts stay.
template <int D, int BS, int CG>
static hipError_t launch_prefill_bs(const PrefillAttnArgs& a, int64_t grid, hipStream_t s) {
  if constexpr (D <= 64 && CG == 2) {
    if (a.wave_groups == 1) {
      hipLaunchKernelGGL((prefill_attn_kernel<D, BS, 1, 8>), dim3((unsigned)grid), dim3(512), 0, s, a);
      return hipGetLastError();
    }
  }
  if (a.wave_groups != CG) return hipErrorInvalidValue;
  hipLaunchKernelGGL((prefill_attn_kernel<D, BS, CG, 4>), dim3((unsigned)grid), dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int D, int CG>
static hipError_t launch_prefill_dc(const PrefillAttnArgs& a, hipStream_t s) {
  const int64_t grid = (int64_t)a.col_blocks * a.max_splits * a.num_seqs * a.hkv;
  return a.bs == 16 ? launch_prefill_bs<D, 16, CG>(a, grid, s) : launch_prefill_bs<D, 0, CG>(a, grid, s);
}

template <int D>
static hipError_t launch_prefill_d(const PrefillAttnArgs& a, hipStream_t s) {
  constexpr int CG = prefill_col_groups(D);
  if constexpr (CG > 1) {
    if (a.col_groups == 1) return launch_prefill_dc<D, 1>(a, s);
  }
  if (a.col_groups != CG) return hipErrorInvalidValue;
  return launch_prefill_dc<D, CG>(a, s);
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
