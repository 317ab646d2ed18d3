// Stream-K paged decode attention for gfx950 (MI355X).
//
// Schedule. The work is a sequence-major list of items, each a run of 16-token
// tiles plus a fixed overhead: the (sequence, kv-head group) pairs, and, where
// neighbouring sequences share leading blocks, one prefix item per (sharing
// group, kv head) placed before the group's first sequence. A persistent grid
// of G workgroups (one per CU, eight wavefronts each) splits the concatenated
// list into G equal contiguous ranges, so every workgroup streams the same
// number of bytes however skewed the sequence lengths are. Every workgroup
// derives the plan itself: its threads load the lengths, find the sharing
// groups, scan the per-sequence widths into LDS and binary-search their
// range's first item.
//
// Shared prefixes. Sequence b joins the group of sequence b - 1 when their
// first table entries are the same physical blocks (up to kPfxCapBlocks
// entries and both sequences' full blocks are compared); a group holds at
// most pfx_members(g) sequences and its shared tiles are the fewest any
// member shares with its predecessor. Its prefix item reads those tiles once
// per kv head and computes the scores of all members' query heads from them
// (four 16-column MFMA blocks), leaving one partial record per member; each
// member's own pairs then cover only the tiles after the prefix. The member's
// output is the log-sum-exp merge of its prefix and suffix records.
//
// Within a range the workgroup walks item segments. Wavefront w takes chunks
// (NT tiles) w, w + 8, w + 16, ... of the segment, keeping an online softmax
// per query head, and the eight wavefronts merge their states through LDS in
// a fixed order at the end of the segment, so results are the same bits on
// every run. A pair wholly inside the range whose sequence shares no prefix is
// written as final fp16 output; every other segment leaves fp32 partial
// records, and the last workgroup to count an arrival for a pair combines the
// pair's records by log-sum-exp, in a fixed order.
//
// Per tile a wavefront loads the K and V rows of HG adjacent kv heads with
// whole-cache-line, non-temporal 16-byte loads (whole contiguous token rows
// when HG * head_dim * 2 bytes is the row), stages them through LDS, computes
// S^T = K Q^T on MFMA for the whole query group of each head (K read back in
// the MFMA operand layout), and O^T += V^T P^T on MFMA with V^T read back
// transposed (see pa_decode.hip for the operand layouts). Block ids are
// fetched three chunks ahead and K/V two chunks ahead of the computation.
#include "pa_tiles.h"

namespace pa {

using namespace tiles;

// Position of workgroup i among n in an order in which each XCD (workgroup i
// runs on XCD i % 8) owns a contiguous run of positions.
__device__ inline int xcd_order(int i, int n) {
  const int n8 = n / kXcds, rem = n % kXcds;
  const int xcd = i % kXcds, k = i / kXcds;
  return xcd * n8 + (xcd < rem ? xcd : rem) + k;
}

// A wavefront-uniform value, moved to a scalar register.
__device__ inline int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// The lane index, computed where it is read and opaque to the compiler: the
// per-lane values a branch derives from it are then formed inside that branch
// instead of being hoisted out of the segment loop and kept live (in vector
// registers) through the other branches' streaming loops.
__device__ inline int fresh_lane() {
  int l = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  asm volatile("" : "+v"(l));
  return l;
}

// First workgroup whose range contains tile x of a T-tile list split G ways.
__host__ __device__ inline int wg_of(int64_t x, int64_t T, int G) {
  return (int)(((x + 1) * G - 1) / T);
}

__host__ __device__ inline int64_t range_start(int w, int64_t T, int G) {
  return (int64_t)w * T / G;
}

// Inclusive prefix sum over the 64 lanes of a wavefront in DPP lane moves:
// shifts by 1, 2, 4 and 8 within each row of 16 lanes (zero shifted in), then
// each row's total broadcast to the rows after it (row_bcast 15 and 31).
__device__ inline int wave_incl_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15 (rows 1, 3)
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31 (rows 2, 3)
  return x;
}

// Exclusive prefix sums over a workgroup of NW wavefronts, PER values per
// thread (thread t holds entries t * PER .. t * PER + PER - 1); returns the
// total. s_tot holds NW ints, written once per call with one barrier: a
// second call reusing s_tot needs a barrier before it. The wavefront scan is
// DPP lane moves with DPP, else six lane shuffles (through LDS): the DPP form
// is shorter, but in some kernels it costs registers their streaming loop
// needs (one more wavefront spill at one kv head per pair, head_dim 64).
template <int PER, int NW, bool DPP>
__device__ inline int block_excl_sum(int (&v)[PER], int* s_tot, int lane, int wave) {
  int local = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) local += v[i];
  int incl = local;
  if constexpr (DPP) {
    incl = wave_incl_scan(local);
  } else {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(incl, off);
      if (lane >= off) incl += y;
    }
  }
  if (lane == 63) s_tot[wave] = incl;
  __syncthreads();
  int run = incl - local, total = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    if (w < wave) run += s_tot[w];
    total += s_tot[w];
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int t = v[i];
    v[i] = run;
    run += t;
  }
  return total;
}

// One wavefront's share of an item segment: tiles s0 .. s1 - 1 (token rows
// 16 ti .. 16 ti + 15 of the sequence whose table row is btrow, length L;
// {s1, L} = seg(), called once the first chunks' block ids are issued where a
// tile lies in one block, so that a length loaded there shares their wait) of
// kv heads h0 .. h0 + HGL - 1, in chunks of NTL tiles w, w + NW, ... (w the
// wavefront). Column block cb of the 16 x 16 score tiles multiplies the query
// fragments qf[cb] with the K rows of kv head h0 + cb, or of kv head h0 for
// every block when SHARED_K (a prefix item: all blocks belong to one kv head).
// Only the first ncb blocks are computed (wavefront-uniform). The online
// softmax state (exp2 domain) accumulates into m_run, l_run and acc. With
// nrow set (LDS: HGL rows of D halves for K, then HGL for V), the rows of
// token L - 1 are taken from nrow instead of the pool: a decode step's new
// token, whose write into the pool need not have landed. pre_loop() runs in
// every wavefront after the first chunks' loads are issued, before any is
// staged or computed (nrow's rows and qf must be complete when it returns;
// nrow is read through the caller's variable, which pre_loop may clear).
struct SegEnd {
  int s1, L;
};
struct KnownSeg {
  static constexpr bool kLoads = false;
  int s1, L;
  __device__ SegEnd operator()() const { return {s1, L}; }
};
struct NoPreLoop {
  __device__ void operator()() const {}
};

template <int D, int BS, int HGL, int NCB, int NTL, bool SHARED_K, int NW, typename Seg,
          typename PreLoop = NoPreLoop>
__device__ __forceinline__ void stream_tiles(const DecodeArgs& a, const int32_t* btrow, int h0,
                                             int s0, Seg seg, int ncb,
                                             const f16x8 (&qf)[NCB][D / 32], f16* kst, f16* vst,
                                             int wave, int lane, float (&m_run)[NCB],
                                             float (&l_run)[NCB], f32x4 (&acc)[NCB][D / 16],
                                             const f16* const& nrow = nullptr,
                                             PreLoop pre_loop = PreLoop{}) {
  constexpr int NC = D / 32;
  constexpr int ND = D / 16;
  constexpr int LS = D + 8;
  constexpr int CPR = HGL * D / 8;  // 16-byte chunks per token row of the loaded heads
  constexpr int NI = 16 * CPR / 64;  // load instructions per tile, for K and for V
  // A 16-token tile lies inside one block when 16 divides the block size: its
  // block id and row base are then wavefront-uniform.
  constexpr bool UNIFORM_TILE = BS > 0 && BS % 16 == 0;
  constexpr int NID = UNIFORM_TILE ? 1 : NI;  // block ids per tile per lane
  constexpr int RS = 64 / CPR;                // token rows one load instruction covers
  static_assert(NI * 64 == 16 * CPR, "tile must split into whole 64-lane loads");
  static_assert(RS * CPR == 64, "a load instruction must cover whole rows");
  static_assert(SHARED_K || NCB == HGL, "one column block per loaded kv head");
  const int row = lane & 15;
  const int grp = lane >> 4;
  const int bs = BS > 0 ? BS : a.bs;
  h0 = uni(h0);  // keeps the tile resources in scalar registers
  int s1 = 0, L = 0;
  if constexpr (!UNIFORM_TILE) {  // the rows' block ids need the length
    const SegEnd e = seg();
    s1 = e.s1;
    L = e.L;
  }
  const int tok_fallback = s0 * 16;  // a valid token of this segment
  const int last_tile = a.max_blocks * (bs / 16) - 1;  // the table's last 16-token tile (uniform tiles)

  // Byte offset of this lane's 16-byte piece within a tile, relative to the
  // tile's first row at the first loaded kv head (same for every tile).
  uint32_t k_lane = 0, v_lane = 0;
  if constexpr (UNIFORM_TILE) {
    const int lrow = lane / CPR, lcol = (lane % CPR) * 8;
    const int lhg = lcol / D, ld0 = lcol - lhg * D;
    k_lane = (uint32_t)(2 * (lrow * a.k_st + lhg * a.k_sh + ld0));
    v_lane = (uint32_t)(2 * (lrow * a.v_st + lhg * a.v_sh + ld0));
  }

  // Natural-layout loads: instruction i of a tile gives lane l the 16-byte
  // chunk f = 64 i + l of the tile's 16 rows x (HGL * D) halves, i.e. row
  // f / CPR, halves (f % CPR) * 8 of the row's head-group slice. Each
  // instruction thus reads whole row slices (whole cache lines).
  auto nat_row = [&](int i) { return (64 * i + lane) / CPR; };
  auto nat_col = [&](int i) { return ((64 * i + lane) % CPR) * 8; };
  auto row_token = [&](int ti, int r) {
    const int t = ti * 16 + r;
    return (ti < s1 && t < L) ? t : tok_fallback;
  };
  auto load_ids = [&](int k, int (&ids)[NTL][NID]) {
#pragma unroll
    for (int nt = 0; nt < NTL; ++nt)
#pragma unroll
      for (int j = 0; j < NID; ++j) {
        // A uniform tile lies in one block; otherwise each lane looks up the
        // block of its own row (also when one instruction covers the tile).
        if constexpr (UNIFORM_TILE) {
          // The tile's entry, clamped to the table width only: no dependence on
          // the length, so the first ids can be in flight with the length
          // itself (a tile past the segment gets an empty resource anyway).
          const int ti = min(s0 + k * NTL + nt, last_tile);
          ids[nt][j] = load_uniform(btrow + (int64_t)(ti / (BS / 16)) * a.bt_sk);
        } else {
          const int t = row_token(s0 + k * NTL + nt, nat_row(j));
          ids[nt][j] = btrow[(int64_t)blk_of<BS>(t, bs) * a.bt_sk];
        }
      }
  };
  auto load_kv = [&](int k, const int (&ids)[NTL][NID], u32x4 (&kb)[NTL][NI],
                     u32x4 (&vb)[NTL][NI]) {
#pragma unroll
    for (int nt = 0; nt < NTL; ++nt) {
      const int ti = s0 + k * NTL + nt;
      if constexpr (UNIFORM_TILE) {
        // Unconditional: a tile past the segment gets an empty resource.
        const int64_t id = min(max(ids[nt][0], 0), a.num_blocks - 1);
        const int64_t r0 = (ti * 16) % BS;
        const int nb = ti < s1 ? 0x7fffffff : 0;
        const auto kr = tile_rsrc(a.k + id * a.k_sb + r0 * a.k_st + (int64_t)h0 * a.k_sh, nb);
        const auto vr = tile_rsrc(a.v + id * a.v_sb + r0 * a.v_st + (int64_t)h0 * a.v_sh, nb);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          kb[nt][i] = load_tile(kr, k_lane, (int)(2 * i * RS * a.k_st));
          vb[nt][i] = load_tile(vr, v_lane, (int)(2 * i * RS * a.v_st));
        }
      } else if (ti < s1) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          const int t = row_token(ti, nat_row(i));
          const int64_t id = min(max(ids[nt][i], 0), a.num_blocks - 1);
          const int64_t off = off_of<BS>(t, bs);
          const int col = nat_col(i);
          const int hg = col / D;
          const int d0 = col - hg * D;
          kb[nt][i] = load_stream(a.k + id * a.k_sb + off * a.k_st + (int64_t)(h0 + hg) * a.k_sh + d0);
          vb[nt][i] = load_stream(a.v + id * a.v_sb + off * a.v_st + (int64_t)(h0 + hg) * a.v_sh + d0);
        }
      }
    }
  };
  // Writes one tile's rows (natural layout) into the staging buffer laid out
  // [tile][head][row][LS]; rows past the sequence end are zeroed when asked.
  auto stage = [&](int k, u32x4 (&buf)[NTL][NI], f16* dst, bool zero_tail, int which) {
#pragma unroll
    for (int nt = 0; nt < NTL; ++nt) {
      const int ti = s0 + k * NTL + nt;
      if (ti < s1) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          const int r = nat_row(i);
          const int col = nat_col(i);
          const int hg = col / D;
          const int d0 = col - hg * D;
          *reinterpret_cast<u32x4*>(&dst[((nt * HGL + hg) * 16 + r) * LS + d0]) = buf[nt][i];
        }
        // Rows past the sequence end are overwritten with zeros in LDS (not
        // selected in registers: a select on freshly loaded registers makes
        // the compiler wait for those loads where it places the select).
        if (zero_tail && ti * 16 + 16 > L) {  // wavefront-uniform: the last tile only
#pragma unroll
          for (int i = 0; i < NI; ++i) {
            const int r = nat_row(i);
            const int col = nat_col(i);
            const int hg = col / D;
            const int d0 = col - hg * D;
            if (ti * 16 + r >= L)
              *reinterpret_cast<f16x8*>(&dst[((nt * HGL + hg) * 16 + r) * LS + d0]) = zero8();
          }
        }
        if (nrow != nullptr && L > 0 && ti == (L - 1) / 16) {  // wavefront-uniform
          // The new token's rows replace what the pool held at its slot.
          const int r = (L - 1) % 16;
          for (int c = lane; c < HGL * D / 8; c += 64) {
            const int hg = c / (D / 8);
            const int d0 = (c - hg * (D / 8)) * 8;
            *reinterpret_cast<f16x8*>(&dst[((nt * HGL + hg) * 16 + r) * LS + d0]) =
                *reinterpret_cast<const f16x8*>(&nrow[(which * HGL + hg) * D + d0]);
          }
        }
      }
    }
  };

  // Both K and V of chunk k go to LDS first, which frees their registers for
  // the loads of the chunk two steps ahead; the math then reads LDS only.
  auto stage_both = [&](int k, u32x4 (&kb)[NTL][NI], u32x4 (&vb)[NTL][NI]) {
    stage(k, kb, kst, false, 0);
    stage(k, vb, vst, true, 1);  // V rows past the sequence end as zeros: 0 * garbage is never NaN
    wave_lds_fence();
  };
  auto compute = [&](int k) {
    float xs[NTL][NCB][4];
    float mloc[NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) mloc[cb] = kNegInf;
#pragma unroll
    for (int nt = 0; nt < NTL; ++nt) {
      const int ti = s0 + k * NTL + nt;
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        if (ti < s1 && cb < ncb) {
          const int kh = SHARED_K ? 0 : cb;
          const f16* kt = kst + ((nt * HGL + kh) * 16 + row) * LS + grp * 8;
          f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < NC; ++c)
            s = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const f16x8*>(kt + 32 * c),
                                                       qf[cb][c], s, 0, 0, 0);
          if (ti * 16 + 16 <= L) {  // wavefront-uniform: only the last tile is partial
#pragma unroll
            for (int r = 0; r < 4; ++r) xs[nt][cb][r] = s[r] * a.scale_log2;
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              xs[nt][cb][r] = ti * 16 + grp * 4 + r < L ? s[r] * a.scale_log2 : kNegInf;
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) mloc[cb] = fmaxf(mloc[cb], xs[nt][cb][r]);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) xs[nt][cb][r] = kNegInf;
        }
      }
    }
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      if (cb < ncb) {
        float m = mloc[cb];
        m = fmaxf(m, __shfl_xor(m, 16));
        m = fmaxf(m, __shfl_xor(m, 32));
        const float m_new = fmaxf(m_run[cb], m);
        const float alpha = fast_exp2(m_run[cb] - m_new);
        l_run[cb] *= alpha;
#pragma unroll
        for (int i = 0; i < ND; ++i) acc[cb][i] *= alpha;
        m_run[cb] = m_new;
      }
    }
    // Probabilities in fp16 high and remainder parts, then O^T += V^T P^T.
    auto probs = [&](int nt, int cb, f16x4& ph, f16x4& pl) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pr = fast_exp2(xs[nt][cb][r] - m_run[cb]);
        l_run[cb] += pr;
        const f16 hi = (f16)pr;
        ph[r] = hi;
        pl[r] = (f16)(pr - (float)hi);
      }
    };
#pragma unroll
    for (int nt = 0; nt < NTL; ++nt) {
      const int ti = s0 + k * NTL + nt;
      if (ti < s1) {
        // V^T operand: lane (row, grp) needs V[4 grp + r][16 nd + row], r = 0..3,
        // which one transposing read of rows 4 grp..4 grp+3 delivers.
        const f16* vt = vst + (nt * HGL * 16 + grp * 4 + (row >> 2)) * LS + (row & 3) * 4;
        if constexpr (SHARED_K) {
          // One V tile for every column block: each transposed read feeds all of them.
          f16x4 ph[NCB], pl[NCB];
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb)
            if (cb < ncb) probs(nt, cb, ph[cb], pl[cb]);
#pragma unroll
          for (int nd = 0; nd < ND; ++nd) {
            const f16x4 av = lds_read_tr16(vt + nd * 16);
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) {
              if (cb < ncb) {
                acc[cb][nd] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, ph[cb], acc[cb][nd], 0, 0, 0);
                acc[cb][nd] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, pl[cb], acc[cb][nd], 0, 0, 0);
              }
            }
          }
        } else {
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb) {
            f16x4 ph, pl;
            probs(nt, cb, ph, pl);
#pragma unroll
            for (int nd = 0; nd < ND; ++nd) {
              const f16x4 av = lds_read_tr16(vt + cb * 16 * LS + nd * 16);
              acc[cb][nd] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, ph, acc[cb][nd], 0, 0, 0);
              acc[cb][nd] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, pl, acc[cb][nd], 0, 0, 0);
            }
          }
        }
      }
    }
    wave_lds_fence();
  };

  // Wavefront-local pipeline over this wavefront's chunks: wavefront w takes
  // chunks w, w + NW, w + 2 NW, ... A fixed assignment (rather than claims
  // from a shared counter, which let faster wavefronts take more chunks) keeps
  // the summation order, and so the result bits, the same on every run; it
  // costs about 1% at large batches. Step s computes chunk c_s: K/V register
  // sets Y0/Y1 hold steps s and s+1, id sets X0/X1 the block ids of steps s+2
  // and s+3. At step s: stage Y[s%2] into LDS, reuse it for the loads of step
  // s+2 (ids in X[s%2]), claim step s+3 and fetch its ids into X[(s+1)%2],
  // then compute step s. Claims are increasing per wavefront, so the first
  // claim past the end ends its work; loads of such chunks are issued anyway
  // (empty resources, clamped table reads) so that no branch separates them.
  int next_chunk = wave;
  auto claim = [&]() {
    const int c = next_chunk;
    next_chunk += NW;
    return c;
  };
  u32x4 kb0[NTL][NI], vb0[NTL][NI], kb1[NTL][NI], vb1[NTL][NI];
  int ids0[NTL][NID], ids1[NTL][NID];
  int c0 = claim();
  int c1 = claim();
  int c2 = claim();
  load_ids(c0, ids0);
  load_ids(c1, ids1);
  if constexpr (UNIFORM_TILE) {
    // Everything issued so far is in flight before the first use of the
    // length: the block ids and a length that seg() loads share one wait.
    if constexpr (Seg::kLoads) __builtin_amdgcn_sched_barrier(0);
    const SegEnd e = seg();
    if constexpr (Seg::kLoads) __builtin_amdgcn_sched_barrier(0);
    s1 = e.s1;
    L = e.L;
  }
  const int nck = __builtin_amdgcn_readfirstlane((s1 - s0 + NTL - 1) / NTL);
  // The scheduler must keep the loads of step 0 ahead of those of step 1:
  // the loop's waits count on the older buffer being the one staged first.
  load_kv(c0, ids0, kb0, vb0);
  __builtin_amdgcn_sched_barrier(0);
  load_kv(c1, ids1, kb1, vb1);
  __builtin_amdgcn_sched_barrier(0);
  load_ids(c2, ids0);
  // The caller's work that may run once the first loads are in flight (every
  // wavefront calls it; it may hold a barrier).
  pre_loop();
  // Two steps per trip, one exit: both steps issue their loads on every trip
  // and only the LDS staging and the math of a step past the end are skipped,
  // so every path through the loop issues the same loads.
  while (c0 < nck) {
    stage_both(c0, kb0, vb0);
    load_kv(c2, ids0, kb0, vb0);
    const int c3 = claim();
    load_ids(c3, ids1);
    compute(c0);
    const bool more = c1 < nck;
    if (more) stage_both(c1, kb1, vb1);
    load_kv(c3, ids1, kb1, vb1);
    const int c4 = claim();
    load_ids(c4, ids0);
    if (more) compute(c1);
    c0 = c2;
    c1 = c3;
    c2 = c4;
  }
}

// Merges the eight wavefronts' states of a segment through LDS (each
// wavefront's area at smem + w * wave_bytes) and hands every merged output
// piece to out(cb, nd, M, den, num): for lane (row, grp), column row of
// column block cb, head_dim elements 16 nd + 4 grp .. + 3, the maximum (exp2
// domain), the denominator and the four unnormalised accumulators. Every
// wavefront stores its maxima and denominators per column block and its
// accumulators in register layout (chunk j = cb * ND + nd: one f32x4 per
// lane, so the 16-byte LDS writes are conflict-free); wavefront w then
// combines chunks j = w, w + NW, ... of all wavefronts, in wavefront order.
template <int D, int NCB, int NW, typename Out>
__device__ __forceinline__ void merge_waves(char* smem, int wave_bytes, int wave, int lane,
                                            const float (&m_run)[NCB], const float (&l_run)[NCB],
                                            const f32x4 (&acc)[NCB][D / 16], int ncb, Out out) {
  constexpr int ND = D / 16;
  const int row = lane & 15;
  const int grp = lane >> 4;
  // A wavefront's state goes to its own area, which held only its own
  // staging buffers: no barrier is needed before these writes.
  float* cm = reinterpret_cast<float*>(smem + wave * wave_bytes);
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    if (cb < ncb) {
      float l = l_run[cb];
      l += __shfl_xor(l, 16);
      l += __shfl_xor(l, 32);
      if (grp == 0) {
        cm[cb * 16 + row] = m_run[cb];
        cm[NCB * 16 + cb * 16 + row] = l;
      }
#pragma unroll
      for (int nd = 0; nd < ND; ++nd)
        *reinterpret_cast<f32x4*>(&cm[32 * NCB + ((cb * ND + nd) * 64 + lane) * 4]) = acc[cb][nd];
    }
  }
  __syncthreads();
  for (int j = wave; j < ncb * ND; j += NW) {
    const int cb = j / ND;
    const int nd = j - cb * ND;
    float mw[NW];
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      mw[w] = reinterpret_cast<const float*>(smem + w * wave_bytes)[cb * 16 + row];
      M = fmaxf(M, mw[w]);
    }
    float den = 0.f;
    f32x4 num = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float* c = reinterpret_cast<const float*>(smem + w * wave_bytes);
      const float sc = mw[w] == kNegInf ? 0.f : fast_exp2(mw[w] - M);
      den += sc * c[NCB * 16 + cb * 16 + row];
      num += sc * *reinterpret_cast<const f32x4*>(&c[32 * NCB + (j * 64 + lane) * 4]);
    }
    out(cb, nd, M, den, num);
  }
}

// The stream-K plan: every sequence's first position in the list of work
// items (prefix items, then pairs, with a segment cost per pair), into s_pos
// (B + 1 entries), and with sharing its group information into s_info. Every
// workgroup of a launch computes the same plan from the lengths and the
// tables' leading columns; the decode layer's K/V write launch can compute it
// once ahead of the attention launch instead. Runs in one workgroup of NW
// wavefronts and ends with a barrier.
template <int NW, bool SHARE, bool DPP_SCAN>
__device__ __forceinline__ void sk_plan(const DecodeArgs& a, const int NHG, int* s_pos,
                                        int* s_info, int* s_wtot) {
  constexpr int NTHR = 64 * NW;
  constexpr int PER = kSkMaxSeqs / NTHR;  // sequences planned per thread
  static_assert(PER * NTHR == kSkMaxSeqs, "plan layout");
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int B = a.num_seqs;
  const int Hkv = a.hkv;
  const int bs = a.bs;
  const bool share = SHARE && a.share;
  // List positions of a prefix item's tiles: one per tile.
  auto pfx_pos = [&](int pt) { return pt; };
  // Every load of the plan is issued before any is used, so that the plan
  // costs one memory round trip: the table rows the sharing groups are found
  // from (below), then the lengths (unconditional, indices clamped; a branch
  // per load would wait for each in turn).
  int rows[32];
  const int capc = min(kPfxCapBlocks, a.max_blocks);
  const int col = min(lane, capc - 1);
  // Rows b0 .. b0 + 31 (clamped to the batch): 32-bit offsets from the
  // slice's first row (the host enables sharing only where 32 rows and 64
  // columns of the table span less than 2^31 entries), so a row costs a min
  // and a 32-bit multiply instead of a 64-bit product.
  auto load_rows = [&](int b0) {
    const int32_t* base = a.bt + (int64_t)b0 * a.bt_sb;
    const int rlast = B - 1 - b0;
    const uint32_t cofs = (uint32_t)col * (uint32_t)a.bt_sk;
#pragma unroll
    for (int r = 0; r < 32; ++r)
      rows[r] = base[(uint32_t)min(r, rlast) * (uint32_t)a.bt_sb + cofs];
  };
  // The sharing compare also needs lane r's length of sequence b0 + r.
  int wlen = 0;
  auto load_wlen = [&](int b0) {
    wlen = a.lens ? a.lens[min(b0 + lane, B - 1)] : a.uniform_len;
  };
  if (share && wave * 32 < B) {
    load_rows(wave * 32);
    load_wlen(wave * 32);
  }
  int Ls[PER];
  if (a.lens) {
#pragma unroll
    for (int i = 0; i < PER; ++i) Ls[i] = a.lens[min(tid * PER + i, B - 1)];
  } else {
#pragma unroll
    for (int i = 0; i < PER; ++i) Ls[i] = a.uniform_len;
  }
  {
    const int cap = a.max_blocks * a.bs;
#pragma unroll
    for (int i = 0; i < PER; ++i)
      Ls[i] = tid * PER + i < B ? min(max(Ls[i], 0), cap) : 0;  // as clamped_len
  }
  if constexpr (SHARE) {
    if (share) {
      // Sharing groups, found by each wavefront for its slices of 32
      // sequences (w * 32 + 256 k ..), with no barrier: lane j holds table
      // entry j of rows b0 .. b0 + 31 and lane r the length of sequence b0 + r;
      // the wavefront finds, per sequence, the leading entries it shares with
      // its predecessor, cuts runs of sharing sequences into groups of at most
      // max_members (a group never crosses a slice) and writes each sequence's
      // group information to s_info.
      for (int b0 = wave * 32; b0 < B; b0 += NW * 32) {
        if (b0 != wave * 32) {
          load_rows(b0);
          load_wlen(b0);
        }
        // Lane r: the table entries sequence b0 + r and its predecessor both
        // hold as full blocks (at most capc).
        const int fl = min(max(wlen, 0), a.max_blocks * a.bs) / bs;
        const int limv = min(capc, min(fl, __shfl_up(fl, 1)));
        // ct: lane i < 32 gets the tiles sequence b0 + i shares with b0 + i - 1
        // (zero for the slice's first sequence: groups start at slice starts).
        // Per sequence one compare into a 64-bit lane mask; its first set bit
        // (the first differing entry, 64 if none) is found in scalar registers,
        // parked in the slice's own s_info entries (overwritten below by this
        // wavefront), read back by lane r and capped at the lane's limit. The
        // 31 compares are independent; capping each in scalar registers and
        // writing it into lane r through inline assembly (a scheduling barrier
        // to the compiler) chained them one after another: about 1.5 us per
        // slice.
        // In four chunks of eight, so that at most eight results are live in
        // scalar registers at once.
#pragma unroll
        for (int r0 = 0; r0 < 32; r0 += 8) {
          int cr[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int r = r0 + i;
            const uint64_t diff = r == 0 ? 0 : __ballot(rows[r] != rows[r > 0 ? r - 1 : 0]);
            cr[i] = diff ? (int)__builtin_ctzll(diff) : 64;
          }
          if (lane == 0) {
#pragma unroll
            for (int i = 0; i < 8; ++i) s_info[b0 + r0 + i] = cr[i];
          }
        }
        wave_lds_fence();
        const int cfirst = lane >= 1 && lane < 32 ? s_info[b0 + lane] : 64;
        wave_lds_fence();
        int ct = lane >= 1 && lane < 32 ? min(min(cfirst, limv) * (bs / 16), 255) : 0;
        const int bl = b0 + lane;  // lane i < 32: sequence b0 + i
        const bool valid = lane < 32 && bl < B;
        if (!valid) ct = 0;
        // Run starts (a sequence sharing nothing with its predecessor; lanes
        // 32 .. 63 count as starts): the last at or before this lane, and the
        // first after it, from one lane mask.
        const uint64_t starts = __ballot(ct == 0);
        const uint64_t upto = starts & (lane == 63 ? ~0ull : (2ull << lane) - 1);
        const int rs = 63 - (int)__builtin_clzll(upto);  // lane 0 is a start: upto != 0
        const uint64_t after = starts & ~(lane == 63 ? ~0ull : (2ull << lane) - 1);
        const int nxt = after ? (int)__builtin_ctzll(after) : 64;
        const int m = (lane - rs) % a.max_members;
        const int gs = min(a.max_members, nxt - lane);  // meaningful at leaders (m == 0)
        int pt = 255;
#pragma unroll
        for (int k = 1; k < kPfxMaxMembers; ++k) {
          const int v = __shfl_down(ct, k);
          if (k < gs) pt = min(pt, v);
        }
        // Shared when the reads it saves outweigh the prefix items' overhead.
        const bool worth = gs > 1 && (int64_t)(gs - 1) * NHG * pt > (int64_t)Hkv * a.seg_cost;
        const int lead = lane - m;
        const int gsl = __shfl(gs, lead);
        const int ptl = __shfl(worth ? pt : 0, lead);
        if (valid) s_info[bl] = ptl ? (ptl | (m << 8) | (gsl << 12)) : 0;
      }
      __syncthreads();
    }
  }
  {
    int cnt[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int b = tid * PER + i;
      const int n = (Ls[i] + 15) >> 4;
      int pt = 0, m = 0;
      if constexpr (SHARE) {
        if (share && b < B) {
          pt = s_info[b] & 255;
          m = (s_info[b] >> 8) & 15;
        }
      }
      // Each pair: its tiles after the shared prefix plus the segment overhead;
      // a group leader also holds the group's prefix items, one per kv head.
      const int w = n - pt > 0 ? n - pt + a.seg_cost : 0;
      cnt[i] = b < B ? NHG * w + (pt > 0 && m == 0 ? Hkv * (pfx_pos(pt) + a.seg_cost) : 0) : 0;
    }
    const int total = block_excl_sum<PER, NW, DPP_SCAN>(cnt, s_wtot, lane, wave);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int b = tid * PER + i;
      if (b < B) s_pos[b] = cnt[i];
    }
    if (tid == 0) s_pos[B] = total;
    __syncthreads();
  }
}

// PLAN_IN: the plan comes from a.plan_in (left by the K/V write launch just
// before this one) instead of being derived by every workgroup.
template <int D, int NT, int BS, int HG, int NW, bool PLAN_IN = false>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2)))
void decode_streamk_kernel(DecodeArgs a) {
  constexpr int NC = D / 32;
  constexpr int ND = D / 16;
  constexpr int LS = D + 8;
  constexpr int NTHR = 64 * NW;
  constexpr bool UNIFORM_TILE = BS > 0 && BS % 16 == 0;
  // Prefix items are built where a tile lies in one block and four column
  // blocks of accumulators fit the registers.
  constexpr bool SHARE = UNIFORM_TILE && D <= 64;
  constexpr int NCP = kPfxColBlocks;
  constexpr int NTP = 2;  // tiles per chunk of a prefix item (one kv head)
  constexpr int VST = NT * HG * 16 * LS;  // halves of one staging buffer (K or V) per wavefront
  constexpr int CMB = 32 * HG + HG * ND * 64 * 4;  // floats of merge state per wavefront
  constexpr int VSTP = SHARE ? NTP * 16 * LS : 0;
  constexpr int CMBP = SHARE ? 32 * NCP + NCP * ND * 64 * 4 : 0;
  // Per wavefront: a K and a V staging buffer; the merge state reuses the same
  // bytes at segment ends.
  constexpr int WAVE_BYTES_0 = 2 * VST * 2 > CMB * 4 ? 2 * VST * 2 : CMB * 4;
  constexpr int WAVE_BYTES_1 = 2 * VSTP * 2 > CMBP * 4 ? 2 * VSTP * 2 : CMBP * 4;
  constexpr int WAVE_BYTES = WAVE_BYTES_0 > WAVE_BYTES_1 ? WAVE_BYTES_0 : WAVE_BYTES_1;
  constexpr int PER = kSkMaxSeqs / NTHR;  // sequences planned per thread
  constexpr int REC = record_floats(D);
  static_assert(PER * NTHR == kSkMaxSeqs, "plan layout");
  __shared__ __attribute__((aligned(16))) char smem[NW * WAVE_BYTES];
  // Sequence -> first list position of its items (prefix items, then pairs).
  __shared__ int s_pos[kSkMaxSeqs + 1];
  // Sequence -> its group's shared tiles (bits 0-7, zero: none), its member
  // index (8-11) and the group's size (12-15).
  __shared__ int s_info[SHARE ? kSkMaxSeqs : 1];
  __shared__ int s_wtot[NW];
  __shared__ int s_nmerge;                // pairs listed for merging
  __shared__ int s_mlist[NTHR];           // pairs whose records this workgroup completed

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int row = lane & 15;
  const int grp = lane >> 4;
  const int B = a.num_seqs;
  const int Hkv = a.hkv;
  const int NHG = Hkv / HG;
  const int bs = BS > 0 ? BS : a.bs;
  const int G = gridDim.x;
  const bool share = SHARE && a.share;
  // List positions of a prefix item's tiles: one per tile. A prefix tile holds
  // one kv head (a pair's tile HG of them), but a prefix wavefront keeps a
  // chunk of NTP one-head tiles in flight where a pair's keeps NT tiles of HG
  // heads, and its four column blocks cost more math per byte: in a
  // bandwidth-saturated launch its bytes take about twice as long each.
  auto pfx_pos = [&](int pt) { return pt; };

  // ---- plan: lengths, sharing groups, the exclusive prefix of list positions ----
  if constexpr (PLAN_IN) {
    // Left by the K/V write launch just before this one on the stream (the
    // same computation, run once instead of in every workgroup).
    for (int i = tid; i <= B; i += NTHR) s_pos[i] = a.plan_in[i];
    if constexpr (SHARE) {
      if (share)
        for (int i = tid; i < B; i += NTHR) s_info[i] = a.plan_in[kSkMaxSeqs + 1 + i];
    }
    __syncthreads();
  } else {
    sk_plan<NW, SHARE, HG == 2>(a, NHG, s_pos, s_info, s_wtot);
  }

  // Plan lookups for sequence b: shared tiles of its group, member index,
  // group size, and the widths of its prefix region (leaders) and pairs.
  struct Geo {
    int base, pw, ws, pt, m, gs;
  };
  auto geo_of = [&](int base, int next, int info) {
    Geo g;
    g.base = base;
    g.pt = info & 255;
    g.m = (info >> 8) & 15;
    g.gs = info >> 12;
    g.pw = (g.pt > 0 && g.m == 0) ? Hkv * (pfx_pos(g.pt) + a.seg_cost) : 0;
    g.ws = (next - g.base - g.pw) / NHG;
    return g;
  };
  // For a wavefront-uniform b (the segment walk): readfirstlane keeps the
  // values in scalar registers, off the vector registers the streaming loop
  // needs.
  auto geo = [&](int b) {
    return geo_of(uni(s_pos[b]), uni(s_pos[b + 1]), share ? uni(s_info[SHARE ? b : 0]) : 0);
  };
  // For a b that differs between the lanes (the merge of completed pairs).
  auto geo_v = [&](int b) {
    return geo_of(s_pos[b], s_pos[b + 1], share ? s_info[SHARE ? b : 0] : 0);
  };

  // Zero-length sequences have no tiles; their rows are written as zeros.
  const int Hq = a.hkv * a.g;
  for (int b = blockIdx.x; b < B; b += G) {
    if (s_pos[b + 1] == s_pos[b] && geo(b).pt == 0) {
      for (int i = tid; i < Hq * D; i += NTHR) {
        const int hq = i / D;
        a.out[(int64_t)b * a.o_sb + (int64_t)hq * a.o_sh + (i - hq * D)] = (f16)0.f;
      }
    }
  }

  // Ranges: at least min_range tile positions each, at most one per
  // workgroup; workgroups beyond them get no range.
  const int T = uni(s_pos[B]);
  const int Gw = (T + a.min_range - 1) / a.min_range;
  const int Ge = (int)(Gw < G ? Gw : G);  // 0 when every sequence is empty

  // The first Ge workgroups take part. Workgroup i is dispatched to XCD i % 8;
  // renumber the Ge of them so that each XCD owns a contiguous run of ranges:
  // neighbouring sequences then run on the same XCD and share its L2, and
  // every XCD gets work when Ge < G.
  if ((int)blockIdx.x >= Ge) return;
  const int wg = xcd_order(blockIdx.x, Ge);
  const int x0 = (int)range_start(wg, T, Ge);
  const int x1 = (int)range_start(wg + 1, T, Ge);  // once per workgroup: 64-bit is fine

  // First item: in the last sequence whose items start at or before x0.
  int b;
  {
    int lo = 0, hi = B - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_pos[mid] <= x0) lo = mid; else hi = mid - 1;
    }
    b = uni(lo);
  }

  char* my_smem = smem + wave * WAVE_BYTES;
  f16* kst = reinterpret_cast<f16*>(my_smem);  // K staging
  // Partial records (float offsets from a.recs): two slots per workgroup
  // (slot 2 w + 1 for the item range w cuts at its end, slot 2 w for the item
  // it continues from earlier ranges), each of slot_recs records (one per kv
  // head of a pair, or per column block of a prefix item); then, for items a
  // range holds whole, per (sequence, kv head): a suffix record of a sharing
  // member's pair (Q) and a prefix record (P: column block cb of the group led
  // by sequence b is sequence b + cb's entry).
  const int SLOT = a.slot_recs * REC;
  const int64_t QBASE = (int64_t)2 * G * SLOT;
  const int64_t PBASE = QBASE + (int64_t)B * Hkv * REC;
  auto slot_base = [&](int w, bool first) { return (int64_t)(2 * w + (first ? 1 : 0)) * SLOT; };
  const auto rec_rsrc = tile_rsrc(a.recs, a.recs_bytes);

  // The ranges wa .. wa + cnt - 1 that an item's tile positions ps .. ps + n - 1
  // span. In 32-bit arithmetic when T * Ge fits (any realistic launch: 64-bit
  // division is a long instruction sequence, and the merge computes this per
  // record list).
  const bool small_list = (int64_t)T * Ge < ((int64_t)1 << 31);
  auto wg_at = [&](int x) {
    return small_list ? (int)((unsigned)((x + 1) * Ge - 1) / (unsigned)T) : wg_of(x, T, Ge);
  };
  auto span = [&](int ps, int n, int& wa, int& cnt) {
    if (n <= 0) {
      wa = 0;
      cnt = 0;
      return;
    }
    wa = wg_at(ps);
    cnt = wg_at(ps + n - 1) - wa + 1;
  };
  // Records that make up pair p's head hh: its suffix records (ns of them from
  // ranges wa_s ..) then its prefix records (np from ranges wa_p ..).
  auto contributions = [&](int p, int hh, Geo& g, int& wa_s, int& ns, int& wa_p, int& np) {
    const int pb = p / NHG;
    const int hg0 = p - pb * NHG;
    g = geo_v(pb);
    span(g.base + g.pw + hg0 * g.ws + a.seg_cost, g.ws - a.seg_cost, wa_s, ns);
    np = 0;
    wa_p = 0;
    if (g.pt > 0) {
      const int wp = pfx_pos(g.pt) + a.seg_cost;
      const int h = hg0 * HG + hh;
      span(s_pos[pb - g.m] + h * wp + a.seg_cost, pfx_pos(g.pt), wa_p, np);
    }
  };

  // Arrivals this workgroup has listed and not yet resolved: thread t < npend
  // listed one for pair s_mlist[t]; for t < ncounted it has also counted it
  // and holds the value its counter increment returned.
  int npend = 0;
  int ncounted = 0;
  int my_old = 0;

  // Counts the listed arrivals not yet counted: every thread waits for its
  // coherent record stores to complete, then each such arrival increments its
  // pair's counter.
  auto count_listed = [&]() {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid >= ncounted && tid < npend)
      my_old = __hip_atomic_fetch_add(a.cnt + s_mlist[tid], 1, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
    ncounted = npend;
  };

  // Resolves the counted arrivals: a pair whose count this workgroup completed
  // is merged here -- its records in a fixed order (suffix ranges, then prefix
  // ranges), by an online log-sum-exp over 16-byte device-coherent loads (each
  // thread four accumulators of one query head, eight records in flight), all
  // such pairs of the workgroup at once -- and its counter is reset to zero
  // for the next launch.
  auto resolve = [&]() {
    count_listed();
    const int tid = wave * 64 + fresh_lane();
    const int my_pair = tid < npend ? s_mlist[tid] : 0;
    if (tid == 0) s_nmerge = 0;
    __syncthreads();
    if (tid < npend) {
      int expect = 0;
#pragma unroll
      for (int hh = 0; hh < HG; ++hh) {
        Geo g;
        int wa_s, ns, wa_p, np;
        contributions(my_pair, hh, g, wa_s, ns, wa_p, np);
        expect += (hh == 0 ? ns : 0) + np;
      }
      if (my_old == expect - 1) s_mlist[atomicAdd(&s_nmerge, 1)] = my_pair;
    }
    __syncthreads();
    const int nmg = s_nmerge;
    constexpr int DQ = D / 4;
    const int per = HG * a.g * DQ;
    const int mpb = 16 / a.g;
    for (int it = tid; it < nmg * per; it += NTHR) {
      // Item: four accumulators (dq) of query head qr of kv head h of one
      // merged pair.
      const int e = it / per;
      int rem = it - e * per;
      const int hh = rem / (a.g * DQ);
      rem -= hh * a.g * DQ;
      const int qr = rem / DQ;
      const int dq = rem - qr * DQ;
      const int p = s_mlist[e];
      const int pb = p / NHG;
      const int h = (p - pb * NHG) * HG + hh;
      Geo g;
      int wa_s, ns, wa_p, np;
      contributions(p, hh, g, wa_s, ns, wa_p, np);
      const int n = ns + np;
      // Record k: a whole suffix or prefix item of a sharing member has its
      // own record; cut items use range slots. A prefix item's record is one
      // of its column blocks, whose 16 rows hold members cb * mpb .. cb * mpb +
      // mpb - 1 times the query group: this member's rows start at rsh.
      const int cbm = g.m / mpb;
      const int rsh = (g.m - cbm * mpb) * a.g;
      auto rec_of = [&](int k) -> int {
        if (k < ns)
          return (int)(ns == 1 ? QBASE + ((int64_t)pb * Hkv + h) * REC
                               : slot_base(wa_s + k, k == 0) + (int64_t)hh * REC);
        const int j = k - ns;
        return (int)(np == 1 ? PBASE + ((int64_t)(pb - g.m + cbm) * Hkv + h) * REC
                             : slot_base(wa_p + j, j == 0) + (int64_t)cbm * REC);
      };
      float M = kNegInf, den = 0.f;
      f32x4 num = {0.f, 0.f, 0.f, 0.f};
      for (int k0 = 0; k0 < n; k0 += 8) {
        float mv[8], lv[8];
        f32x4 av[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          // Padding past the item's records reads at an offset past the record
          // area: the buffer returns zeros and touches no memory.
          const bool live = k0 + k < n;
          const int kk = live ? k0 + k : 0;
          const int base = rec_of(kk);
          const int r = (kk < ns ? 0 : rsh) + qr;  // this query head's row of the record
          constexpr int kOut = 0x7ffffff0;
          mv[k] = load_coherent4(rec_rsrc, live ? 4 * (base + r) : kOut);
          lv[k] = load_coherent4(rec_rsrc, live ? 4 * (base + 16 + r) : kOut);
          av[k] = load_coherent16(rec_rsrc, live ? 4 * (base + 32 + r * D + dq * 4) : kOut);
          if (!live) mv[k] = kNegInf;
        }
        float mb = M;
#pragma unroll
        for (int k = 0; k < 8; ++k) mb = fmaxf(mb, mv[k]);
        const float sc = M == kNegInf ? 0.f : fast_exp2(M - mb);
        num *= sc;
        den *= sc;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float wk = mv[k] == kNegInf ? 0.f : fast_exp2(mv[k] - mb);
          num += wk * av[k];
          den += wk * lv[k];
        }
        M = mb;
      }
      const float inv = den > 0.f ? 1.f / den : 0.f;
      f16x4 ov;
#pragma unroll
      for (int c = 0; c < 4; ++c) ov[c] = (f16)(num[c] * inv);
      *reinterpret_cast<f16x4*>(a.out + (int64_t)pb * a.o_sb +
                                (int64_t)(h * a.g + qr) * a.o_sh + dq * 4) = ov;
    }
    for (int e = tid; e < nmg; e += NTHR)
      __hip_atomic_store(a.cnt + s_mlist[e], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    npend = 0;
    ncounted = 0;
  };

  // Lists a segment's arrival for each of the n pairs pair_of(i) its records
  // belong to (thread npend + i holds pair i). A pair segment's arrival is
  // counted later, when the workgroup next counts or resolves: its record
  // stores then complete while the next segment streams, instead of holding
  // up that segment's start. The returned counts are only needed when the
  // workgroup resolves its arrivals.
  auto list_arrival = [&](int n, auto pair_of) {
    if (tid >= npend && tid < npend + n) s_mlist[tid] = pair_of(tid - npend);
    npend += n;
  };
  // Lists and counts at once (with every arrival listed before): a prefix
  // item's records complete the counts of its group's members, whose pairs
  // are spread over other workgroups and should merge as soon as they can.
  auto arrive = [&](int n, auto pair_of) {
    list_arrival(n, pair_of);
    count_listed();
  };

  // Item containing list position x (in sequence b's items): kind (0 pair,
  // 1 prefix item), index (kv-head group, or kv head), and its positions.
  auto locate = [&](int bb, int x, int& kind, int& idx, int& is, int& ie, Geo& g) {
    g = geo(bb);
    const int o = x - g.base;
    if (o < g.pw) {
      const int wp = g.pw / Hkv;
      kind = 1;
      idx = o / wp;
      is = g.base + idx * wp;
      ie = is + wp;
    } else {
      kind = 0;
      idx = (o - g.pw) / g.ws;
      is = g.base + g.pw + idx * g.ws;
      ie = is + g.ws;
    }
  };

  // Segment order. The range's prefix-item segments go first (step 0), so
  // that the prefix records are complete early and the members' own segments
  // -- spread over many workgroups -- complete their counts and merge; a prefix
  // item finished last would leave one workgroup merging its whole group at
  // the end of the launch. Then the pairs (steps 1 and 2): a range starts with
  // at most one segment that continues an item begun in an earlier range; it
  // is processed last, so every workgroup starts on the first tiles of a pair:
  // the leading blocks of all sequences -- where sequences share prefix blocks
  // that no prefix item covers -- are read close together in time and repeated
  // reads find them in the L2 / MALL.
  const int b_first = b;
  int cont_end = x0;  // end of the leading continuation segment (x0 if none)
  {
    int kind, idx;
    int is, ie;
    Geo g;
    locate(b, x0, kind, idx, is, ie, g);
    if (is < x0) cont_end = ie < x1 ? ie : x1;
  }
  const int b_cont = b;
  if (cont_end > x0 && cont_end < x1 && cont_end >= uni(s_pos[b + 1])) {
    ++b;
    while (b < B - 1 && uni(s_pos[b + 1]) == uni(s_pos[b])) ++b;
  }

  const int b_pairs = b;
  for (int step = share ? 0 : 1; step < 3; ++step) {
  const int want_kind = step == 0 ? 1 : 0;
  int x = step == 0 ? x0 : (step == 1 ? cont_end : x0);
  const int x_end = step == 0 ? x1 : (step == 1 ? x1 : cont_end);
  b = step == 0 ? b_first : (step == 1 ? b_pairs : b_cont);
  while (x < x_end) {
    // Room for this segment's arrivals in the pending list.
    if (npend > NTHR - kPfxMaxMembers - HG) resolve();
    int kind, idx;
    int pstart, pend;
    Geo g;
    locate(b, x, kind, idx, pstart, pend, g);
    // Segment bounds in the item's tile positions (its first seg_cost
    // positions stand for its fixed overhead and hold no tiles),
    // wavefront-uniform by construction; readfirstlane makes that visible to
    // the compiler, so the loops keep uniform branches (a branch it must treat
    // as divergent gets restructured into paths that skip loads, which spoils
    // the wait counts of the load pipeline).
    const int r0 = uni(max(x - pstart - a.seg_cost, 0));
    const int r1 = uni(max((x1 < pend ? x1 : pend) - pstart - a.seg_cost, 0));
    const bool first = r0 == 0;
    const bool last = pend <= x1;
    if (r1 > r0 && kind == 0 && want_kind == 0) {
      // ---- a pair: kv heads h0 .. h0 + HG - 1 of sequence b, tiles after its prefix ----
      const int lane = fresh_lane();
      const int row = lane & 15, grp = lane >> 4;
      const int L = __builtin_amdgcn_readfirstlane(clamped_len(a, b));
      const int h0 = idx * HG;
      const int s0 = g.pt + r0, s1 = g.pt + r1;
      const bool whole = first && last;
      f16x8 qf[HG][NC];
      {
        const int gq = min(row, a.g - 1);
#pragma unroll
        for (int hg = 0; hg < HG; ++hg) {
          const f16* qp = a.q + (int64_t)b * a.q_sb + (int64_t)((h0 + hg) * a.g + gq) * a.q_sh + grp * 8;
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const f16x8 t = *reinterpret_cast<const f16x8*>(qp + 32 * c);
            qf[hg][c] = row < a.g ? t : zero8();
          }
        }
      }
      float m_run[HG], l_run[HG];
      f32x4 acc[HG][ND];
#pragma unroll
      for (int hg = 0; hg < HG; ++hg) {
        m_run[hg] = kNegInf;
        l_run[hg] = 0.f;
#pragma unroll
        for (int i = 0; i < ND; ++i) acc[hg][i] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      stream_tiles<D, BS, HG, HG, NT, false, NW>(a, a.bt + (int64_t)b * a.bt_sb, h0, s0,
                                                 KnownSeg{s1, L}, HG, qf, kst, kst + VST, wave,
                                                 lane, m_run, l_run, acc);
      const bool final_out = whole && g.pt == 0;
      merge_waves<D, HG, NW>(smem, WAVE_BYTES, wave, lane, m_run, l_run, acc, HG,
                             [&](int hg, int nd, float M, float den, f32x4 num) {
        if (row < a.g) {
          if (final_out) {
            const float inv = den > 0.f ? 1.f / den : 0.f;
            f16x4 o;
#pragma unroll
            for (int r = 0; r < 4; ++r) o[r] = (f16)(num[r] * inv);
            *reinterpret_cast<f16x4*>(a.out + (int64_t)b * a.o_sb +
                                      (int64_t)((h0 + hg) * a.g + row) * a.o_sh + nd * 16 + grp * 4) = o;
          } else {
            const int rb = (int)(whole ? QBASE + ((int64_t)b * Hkv + h0 + hg) * REC
                                       : slot_base(wg, first) + (int64_t)hg * REC);
            if (grp == 0 && nd == 0) {
              store_coherent(a.recs + rb + row, M);
              store_coherent(a.recs + rb + 16 + row, den);
            }
            store_coherent16(rec_rsrc, 4 * (rb + 32 + row * D + nd * 16 + grp * 4), num);
          }
        }
      });
      if (!final_out) {
        const int p = b * NHG + idx;
        list_arrival(1, [&](int) { return p; });
      }
      __syncthreads();  // the merge state aliases the staging buffers of the next segment
    }
    if constexpr (SHARE) {
      if (r1 > r0 && kind == 1 && want_kind == 1) {
        // ---- a prefix item: kv head h, the shared tiles of the group led by b ----
        const int lane = fresh_lane();
        const int row = lane & 15, grp = lane >> 4;
        const int L = __builtin_amdgcn_readfirstlane(clamped_len(a, b));
        const int h = idx;
        const int s0 = r0, s1 = r1;
        const int mpb = 16 / a.g;  // members per column block
        const int gs = g.gs;
        const int ncb = __builtin_amdgcn_readfirstlane((gs + mpb - 1) / mpb);
        const bool whole = first && last;
        // Column row of block cb: query head row % g of member cb * mpb + row / g.
        const int mrow = row / a.g, qh = row - mrow * a.g;
        const bool col_ok = mrow < mpb;
        f16x8 qf[NCP][NC];
#pragma unroll
        for (int cb = 0; cb < NCP; ++cb) {
          const int mm = cb * mpb + mrow;
          const bool ok = col_ok && mm < gs;
          const f16* qp = a.q + (int64_t)(b + (ok ? mm : 0)) * a.q_sb +
                          (int64_t)(h * a.g + qh) * a.q_sh + grp * 8;
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const f16x8 t = *reinterpret_cast<const f16x8*>(qp + 32 * c);
            qf[cb][c] = ok ? t : zero8();
          }
        }
        float m_run[NCP], l_run[NCP];
        f32x4 acc[NCP][ND];
#pragma unroll
        for (int cb = 0; cb < NCP; ++cb) {
          m_run[cb] = kNegInf;
          l_run[cb] = 0.f;
#pragma unroll
          for (int i = 0; i < ND; ++i) acc[cb][i] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        stream_tiles<D, BS, 1, NCP, NTP, true, NW>(a, a.bt + (int64_t)b * a.bt_sb, h, s0,
                                                   KnownSeg{s1, L}, ncb, qf, kst, kst + VSTP, wave,
                                                   lane, m_run, l_run, acc);
        merge_waves<D, NCP, NW>(smem, WAVE_BYTES, wave, lane, m_run, l_run, acc, ncb,
                                [&](int cb, int nd, float M, float den, f32x4 num) {
          // Column block cb is one record: row = column (member, query head).
          if (col_ok && cb * mpb + mrow < gs) {
            const int rb = (int)(whole ? PBASE + ((int64_t)(b + cb) * Hkv + h) * REC
                                       : slot_base(wg, first) + (int64_t)cb * REC);
            if (grp == 0 && nd == 0) {
              store_coherent(a.recs + rb + row, M);
              store_coherent(a.recs + rb + 16 + row, den);
            }
            store_coherent16(rec_rsrc, 4 * (rb + 32 + row * D + nd * 16 + grp * 4), num);
          }
        });
        const int hq = h / HG;
        arrive(gs, [&](int i) { return (b + i) * NHG + hq; });
        __syncthreads();  // the merge state aliases the staging buffers of the next segment
      }
    }
    x = pend;
    if (x < x_end && x >= uni(s_pos[b + 1])) {
      ++b;
      while (b < B - 1 && uni(s_pos[b + 1]) == uni(s_pos[b])) ++b;
    }
  }
  }

  // ---- pairs whose arrivals this workgroup completed: merge their records ----
  resolve();
}

// Rotary embedding of the new token's q or key in fp16, op by op as
// transformers' apply_rotary_pos_emb computes it (every product and sum
// rounded on its own; no fused multiply-add): for element j of the first half
// (x1, partner x2 = element j + D/2, cos and sin at j for o1 and at j + D/2
// for o2)
//   o1 = fp16(fp16(x1 * c1) + fp16(-x2 * s1)),  o2 = fp16(fp16(x2 * c2) + fp16(x1 * s2)).
// The same statement as rope_kv_write_kernel, so both give the same bits. The
// inputs are taken by value: the outputs may be the inputs' own variables.
__device__ __forceinline__ void rope8(const f16x8 x1, const f16x8 x2, const f16x8 c1,
                                      const f16x8 c2, const f16x8 s1, const f16x8 s2,
                                      f16x8& o1, f16x8& o2) {
#pragma clang fp contract(off)
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const f16 a1 = x1[e] * c1[e];
    const f16 b1 = -(x2[e] * s1[e]);
    o1[e] = a1 + b1;
    const f16 a2 = x2[e] * c2[e];
    const f16 b2 = x1[e] * s2[e];
    o2[e] = a2 + b2;
  }
}

// The pair kernel's segment end: the whole sequence, its length loaded where
// stream_tiles asks for it (and kept in L_out for the rest of the kernel).
struct PairSeg {
  static constexpr bool kLoads = true;
  const int32_t* len;  // nullptr: every sequence has uniform_len tokens
  int uniform_len, cap;
  int& L_out;
  int& Lraw_out;  // the length as given (a write past the table is skipped)
  __device__ SegEnd operator()() const {
    const int Lraw = len ? load_uniform(len) : uniform_len;
    const int L = min(max(Lraw, 0), cap);
    Lraw_out = Lraw;
    L_out = L;
    return {(L + 15) >> 4, L};
  }
};

// Batched decode with one workgroup per (sequence, kv-head group) pair, for
// batches whose pairs fill the GPU and are short (the schedule the C API
// picks for them): no plan and no partial records. Workgroup w takes pair w
// (in XCD order); its first memory round trip brings the sequence's length,
// the block ids of its first chunks, the query rows and, with ROPE, the new
// token's key and value rows and the rotary cos / sin rows.
//
// NEWROW 2, ROPE (the fused decode-layer form): q and the new key arrive
// unrotated; the kernel rotates them (rope8), attends over the L tokens with
// the new token's rotated key and value substituted for the pool's rows at
// position L - 1, and writes them into that slot of the pool -- the work of
// rope_kv_write_kernel followed by this kernel without it, in one launch. The
// write is issued at the end: no workgroup but this one reads the pair's
// rows during the launch. NEWROW 1: the same without the rotation (the K/V
// write followed by this kernel); NEWROW 0: attention only.
template <int D, int NT, int BS, int HG, int NW, int NEWROW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2)))
void decode_pair_kernel(DecodeArgs a, RopeIn r) {
  constexpr bool ROPE = NEWROW == 2;
  constexpr bool WRITE = NEWROW != 0;
  constexpr int NC = D / 32;
  constexpr int ND = D / 16;
  constexpr int LS = D + 8;
  constexpr int VST = NT * HG * 16 * LS;
  constexpr int CMB = 32 * HG + HG * ND * 64 * 4;
  constexpr int WAVE_BYTES = 2 * VST * 2 > CMB * 4 ? 2 * VST * 2 : CMB * 4;
  static_assert(!ROPE || D >= 64, "rotation pairs must lie in one lane's query fragments");
  __shared__ __attribute__((aligned(16))) char smem[NW * WAVE_BYTES];
  __shared__ __attribute__((aligned(16))) f16 s_new[WRITE ? 2 * HG * D : 8];  // new K rows, then V rows

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int row = lane & 15;
  const int grp = lane >> 4;
  const int NHG = a.hkv / HG;
  const int P = a.num_seqs * NHG;
  if ((int)blockIdx.x >= P) return;
  const int wg = xcd_order(blockIdx.x, P);
  const int b = wg / NHG;
  const int h0 = (wg - b * NHG) * HG;

  // Query fragments (with ROPE, element j of the first half and its partner
  // j + D / 2 sit in fragments c and c + NC / 2 of the same lane). Only their
  // loads are issued here; the rotation waits for the pipeline's first loads.
  f16x8 qf[HG][NC];
  f16x8 qc[ROPE ? NC : 1], qs[ROPE ? NC : 1];
  {
    const int gq = min(row, a.g - 1);
#pragma unroll
    for (int hg = 0; hg < HG; ++hg) {
      const f16* qp = a.q + (int64_t)b * a.q_sb + (int64_t)((h0 + hg) * a.g + gq) * a.q_sh + grp * 8;
#pragma unroll
      for (int c = 0; c < NC; ++c) qf[hg][c] = *reinterpret_cast<const f16x8*>(qp + 32 * c);
    }
    if constexpr (ROPE) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        qc[c] = *reinterpret_cast<const f16x8*>(r.cos + (int64_t)b * r.cs_b + grp * 8 + 32 * c);
        qs[c] = *reinterpret_cast<const f16x8*>(r.sin + (int64_t)b * r.ss_b + grp * 8 + 32 * c);
      }
    } else {
#pragma unroll
      for (int hg = 0; hg < HG; ++hg)
#pragma unroll
        for (int c = 0; c < NC; ++c)
          if (row >= a.g) qf[hg][c] = zero8();
    }
  }

  // WRITE: the new token's key and value rows. Lane t < HG * D / 16 of the
  // first wavefront takes 8 elements j of one head and their partners
  // j + D / 2; the key (rotated with ROPE) and the value go to s_new.
  constexpr int NRL = HG * D / 16;
  f16x8 nk1, nk2, nv1, nv2, nc1, nc2, ns1, ns2;
  if constexpr (WRITE) {
    if (tid < NRL) {
      const int hg = tid / (D / 16);
      const int j = (tid - hg * (D / 16)) * 8;
      const f16* kp = r.key + (int64_t)b * r.ks_b + (int64_t)(h0 + hg) * r.ks_h;
      const f16* vp = r.val + (int64_t)b * r.vs_b + (int64_t)(h0 + hg) * r.vs_h;
      nk1 = *reinterpret_cast<const f16x8*>(kp + j);
      nk2 = *reinterpret_cast<const f16x8*>(kp + j + D / 2);
      nv1 = *reinterpret_cast<const f16x8*>(vp + j);
      nv2 = *reinterpret_cast<const f16x8*>(vp + j + D / 2);
      if constexpr (ROPE) {
        const f16* cp = r.cos + (int64_t)b * r.cs_b;
        const f16* sp = r.sin + (int64_t)b * r.ss_b;
        nc1 = *reinterpret_cast<const f16x8*>(cp + j);
        nc2 = *reinterpret_cast<const f16x8*>(cp + j + D / 2);
        ns1 = *reinterpret_cast<const f16x8*>(sp + j);
        ns2 = *reinterpret_cast<const f16x8*>(sp + j + D / 2);
      }
    }
  }
  // The length is loaded after the first block ids are issued (they do not
  // depend on it), so that both arrive in one round trip. A sequence with no
  // tokens streams no tile: every wavefront keeps an empty state and the
  // merge writes rows of zeros.
  int L = 0;
  int Lraw = 0;
  // The rows substituted for the pool's at position L - 1; cleared when the
  // given length puts the new token's slot past the table (no write then, as
  // in rope_kv_write_kernel, so the pool's row is read).
  const f16* nrow = WRITE ? s_new : nullptr;
  // Runs in every wavefront once the first chunks' loads are in flight (the
  // length known): with WRITE it also fetches the block id of the new token's
  // slot, position L - 1, for the write at the end.
  int slot_id = -1;
  auto rotate = [&]() {
    if constexpr (WRITE) {
      const int lb = (L - 1) / a.bs;
      if (Lraw > a.max_blocks * a.bs) nrow = nullptr;
      else if (L > 0 && lb < a.max_blocks)
        slot_id = load_uniform(a.bt + (int64_t)b * a.bt_sb + (int64_t)lb * a.bt_sk);
      if constexpr (ROPE) {
#pragma unroll
        for (int hg = 0; hg < HG; ++hg) {
#pragma unroll
          for (int c = 0; c < NC / 2; ++c)
            rope8(qf[hg][c], qf[hg][c + NC / 2], qc[c], qc[c + NC / 2], qs[c], qs[c + NC / 2],
                  qf[hg][c], qf[hg][c + NC / 2]);
#pragma unroll
          for (int c = 0; c < NC; ++c)
            if (row >= a.g) qf[hg][c] = zero8();
        }
      }
      if (tid < NRL) {
        const int hg = tid / (D / 16);
        const int j = (tid - hg * (D / 16)) * 8;
        if constexpr (ROPE) rope8(nk1, nk2, nc1, nc2, ns1, ns2, nk1, nk2);
        *reinterpret_cast<f16x8*>(&s_new[hg * D + j]) = nk1;
        *reinterpret_cast<f16x8*>(&s_new[hg * D + j + D / 2]) = nk2;
        *reinterpret_cast<f16x8*>(&s_new[(HG + hg) * D + j]) = nv1;
        *reinterpret_cast<f16x8*>(&s_new[(HG + hg) * D + j + D / 2]) = nv2;
      }
      __syncthreads();
    }
  };

  PairSeg seg{a.lens ? a.lens + b : nullptr, a.uniform_len, a.max_blocks * a.bs, L, Lraw};

  f16* kst = reinterpret_cast<f16*>(smem + wave * WAVE_BYTES);
  float m_run[HG], l_run[HG];
  f32x4 acc[HG][ND];
#pragma unroll
  for (int hg = 0; hg < HG; ++hg) {
    m_run[hg] = kNegInf;
    l_run[hg] = 0.f;
#pragma unroll
    for (int i = 0; i < ND; ++i) acc[hg][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  stream_tiles<D, BS, HG, HG, NT, false, NW>(a, a.bt + (int64_t)b * a.bt_sb, h0, 0, seg, HG, qf,
                                             kst, kst + VST, wave, lane, m_run, l_run, acc,
                                             nrow, rotate);
  merge_waves<D, HG, NW>(smem, WAVE_BYTES, wave, lane, m_run, l_run, acc, HG,
                         [&](int hg, int nd, float, float den, f32x4 num) {
    if (row < a.g) {
      const float inv = den > 0.f ? 1.f / den : 0.f;
      f16x4 o;
#pragma unroll
      for (int q = 0; q < 4; ++q) o[q] = (f16)(num[q] * inv);
      *reinterpret_cast<f16x4*>(a.out + (int64_t)b * a.o_sb +
                                (int64_t)((h0 + hg) * a.g + row) * a.o_sh + nd * 16 + grp * 4) = o;
    }
  });

  if constexpr (WRITE) {
    // The new token's slot: position L - 1, in the block the table lists for
    // it; a slot outside the table or the pool is not written (as in
    // rope_kv_write_kernel), nor is anything for a sequence with no tokens.
    if (tid < NRL && L > 0 && nrow != nullptr) {
      const int pos = L - 1;
      const int lb = pos / a.bs;
      const int id = slot_id;
      if (id >= 0 && id < a.num_blocks) {
        const int hg = tid / (D / 16);
        const int j = (tid - hg * (D / 16)) * 8;
        const int64_t off = (int64_t)(pos - lb * a.bs);
        f16* kd = const_cast<f16*>(a.k) + (int64_t)id * a.k_sb + off * a.k_st + (int64_t)(h0 + hg) * a.k_sh;
        f16* vd = const_cast<f16*>(a.v) + (int64_t)id * a.v_sb + off * a.v_st + (int64_t)(h0 + hg) * a.v_sh;
        *reinterpret_cast<f16x8*>(kd + j) = *reinterpret_cast<const f16x8*>(&s_new[hg * D + j]);
        *reinterpret_cast<f16x8*>(kd + j + D / 2) = *reinterpret_cast<const f16x8*>(&s_new[hg * D + j + D / 2]);
        *reinterpret_cast<f16x8*>(vd + j) = *reinterpret_cast<const f16x8*>(&s_new[(HG + hg) * D + j]);
        *reinterpret_cast<f16x8*>(vd + j + D / 2) = *reinterpret_cast<const f16x8*>(&s_new[(HG + hg) * D + j + D / 2]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Launchers.
// ---------------------------------------------------------------------------
namespace {

constexpr int kSkWaves = 8;

// Tiles per chunk: two chunks of K/V (one computing, one in flight) must fit
// the 256 VGPRs a wavefront has at two wavefronts per SIMD. From head_dim 64
// on, one tile per chunk: a pair's tiles spread over more wavefronts and each
// step waits for less. Measured on MI355X (HIP events behind a GPU busy-wait,
// medians of 60 calls) against two tiles: the batch-128 decode layer 14.4 vs
// 15.6 us, with RoPE and the K/V write 14.7 vs 16.0; batch 1-32 x 512-1024
// tokens 0.6-1.3 us faster; 32 x 2048 18.8 vs 19.9; batch 64 x 2048 at head_dim
// 128, 4/7/28 kv heads, 1.4-2.6% faster; the headline batch (two kv heads per
// pair) unchanged. Four tiles: 1.7-3.5 us slower at those small batches; three
// one-tile chunks in flight per wavefront instead of two: 0.5-1.1 us slower.
template <int D>
constexpr int sk_chunk_tiles(int hg) {
  return D <= 32 ? (hg == 2 ? 2 : 4) : 1;
}

template <int D, int BS, int HG>
hipError_t launch_sk(const DecodeArgs& a, hipStream_t s) {
  constexpr int NT = sk_chunk_tiles<D>(HG);
  if (a.pair_per_wg)
    decode_pair_kernel<D, NT, BS, HG, kSkWaves, 0><<<a.num_wg, 64 * kSkWaves, 0, s>>>(a, RopeIn{});
  else
    decode_streamk_kernel<D, NT, BS, HG, kSkWaves><<<a.num_wg, 64 * kSkWaves, 0, s>>>(a);
  return hipGetLastError();
}

template <int D, int BS, int HG>
hipError_t launch_sk_plan_in(const DecodeArgs& a, hipStream_t s) {
  constexpr int NT = sk_chunk_tiles<D>(HG);
  decode_streamk_kernel<D, NT, BS, HG, kSkWaves, true><<<a.num_wg, 64 * kSkWaves, 0, s>>>(a);
  return hipGetLastError();
}

template <int D, int BS, int HG>
hipError_t launch_pair_rope(const DecodeArgs& a, const RopeIn& r, hipStream_t s) {
  constexpr int NT = sk_chunk_tiles<D>(HG);
  decode_pair_kernel<D, NT, BS, HG, kSkWaves, 2><<<a.num_wg, 64 * kSkWaves, 0, s>>>(a, r);
  return hipGetLastError();
}

// Attention with the new token's K/V write in the same launch (one workgroup
// per pair).
template <int D, int BS, int HG>
hipError_t launch_write(const DecodeArgs& a, const RopeIn& r, hipStream_t s) {
  constexpr int NT = sk_chunk_tiles<D>(HG);
  decode_pair_kernel<D, NT, BS, HG, kSkWaves, 1><<<a.num_wg, 64 * kSkWaves, 0, s>>>(a, r);
  return hipGetLastError();
}

// The block-size-specialised kernels address a tile's K/V through a buffer
// resource with 32-bit offsets: every byte offset inside a 16-row tile must
// stay below 2^31. Pools with larger strides take the generic kernel.
inline bool tile_offsets_fit(const DecodeArgs& a, int D, int HG) {
  auto span = [&](int64_t st, int64_t sh) { return 2 * (15 * st + (HG - 1) * sh + D); };
  const int64_t lim = (int64_t)1 << 31;
  return a.k_st >= 0 && a.k_sh >= 0 && a.v_st >= 0 && a.v_sh >= 0 &&
         span(a.k_st, a.k_sh) < lim && span(a.v_st, a.v_sh) < lim;
}

template <int D, int HG>
hipError_t launch_sk_bs(const DecodeArgs& a, hipStream_t s) {
  if (!tile_offsets_fit(a, D, HG)) return launch_sk<D, 0, HG>(a, s);
  switch (a.bs) {
    case 8: return launch_sk<D, 8, HG>(a, s);
    case 16: return launch_sk<D, 16, HG>(a, s);
    case 32: return launch_sk<D, 32, HG>(a, s);
    default: return launch_sk<D, 0, HG>(a, s);
  }
}

}  // namespace

// Whether the kernel launched for these arguments builds prefix items (the
// host sizes the workspace and sets a.share only then).
bool streamk_can_share(const DecodeArgs& a, int D) {
  // The plan reads 32 rows and kPfxCapBlocks columns of the table per slice
  // with 32-bit offsets.
  const bool table_fits = a.bt_sb >= 0 && a.bt_sk >= 0 &&
                          a.bt_sb * 31 + a.bt_sk * (kPfxCapBlocks - 1) < ((int64_t)1 << 31);
  return D <= 64 && (a.bs == 16 || a.bs == 32) && tile_offsets_fit(a, D, a.head_group) &&
         table_fits;
}

bool pair_rope_supported(const DecodeArgs& a, int D) {
  return a.pair_per_wg && (D == 64 || D == 128) && (a.bs == 16 || a.bs == 32) &&
         tile_offsets_fit(a, D, a.head_group) && (a.head_group == 1 || D == 64);
}

hipError_t launch_decode_pair_rope(const DecodeArgs& a, const RopeIn& r, int D, hipStream_t s) {
  if (!pair_rope_supported(a, D)) return hipErrorInvalidValue;
  if (D == 64) {
    if (a.head_group == 2)
      return a.bs == 16 ? launch_pair_rope<64, 16, 2>(a, r, s) : launch_pair_rope<64, 32, 2>(a, r, s);
    return a.bs == 16 ? launch_pair_rope<64, 16, 1>(a, r, s) : launch_pair_rope<64, 32, 1>(a, r, s);
  }
  return a.bs == 16 ? launch_pair_rope<128, 16, 1>(a, r, s) : launch_pair_rope<128, 32, 1>(a, r, s);
}

bool decode_write_supported(const DecodeArgs& a, int D) {
  return a.pair_per_wg && (D == 64 || D == 128) && (a.bs == 16 || a.bs == 32) &&
         tile_offsets_fit(a, D, a.head_group) && (a.head_group == 1 || D == 64);
}

hipError_t launch_decode_write(const DecodeArgs& a, const RopeIn& r, int D, hipStream_t s) {
  if (!decode_write_supported(a, D)) return hipErrorInvalidValue;
  if (D == 64) {
    if (a.head_group == 2)
      return a.bs == 16 ? launch_write<64, 16, 2>(a, r, s) : launch_write<64, 32, 2>(a, r, s);
    return a.bs == 16 ? launch_write<64, 16, 1>(a, r, s) : launch_write<64, 32, 1>(a, r, s);
  }
  return a.bs == 16 ? launch_write<128, 16, 1>(a, r, s) : launch_write<128, 32, 1>(a, r, s);
}

// The decode layer's K/V write together with the stream-K plan of the
// attention launch that follows it on the stream: workgroup 0 derives the
// plan (the computation every attention workgroup would otherwise repeat)
// and leaves it at a.plan_out; the other workgroups copy the new rows. The
// attention launch starts once this one has ended, so it reads the plan and
// the pool rows complete.
template <int NW, bool VEC>
__global__ __launch_bounds__(64 * NW) void kv_write_plan_kernel(DecodeArgs a, KVWriteArgs w) {
  if (blockIdx.x == 0) {
    __shared__ int s_pos[kSkMaxSeqs + 1];
    __shared__ int s_info[kSkMaxSeqs];
    __shared__ int s_wtot[NW];
    sk_plan<NW, true, true>(a, a.hkv / a.head_group, s_pos, s_info, s_wtot);
    for (int i = threadIdx.x; i <= a.num_seqs; i += 64 * NW) a.plan_out[i] = s_pos[i];
    if (a.share)
      for (int i = threadIdx.x; i < a.num_seqs; i += 64 * NW)
        a.plan_out[kSkMaxSeqs + 1 + i] = s_info[i];
    return;
  }
  kv_write_rows<VEC>(w, (int64_t)(blockIdx.x - 1) * blockDim.x + threadIdx.x,
                     (int64_t)(gridDim.x - 1) * blockDim.x);
}

bool plan_handover_supported(const DecodeArgs& a, int D) {
  return !a.pair_per_wg && a.num_seqs <= kSkMaxSeqs && (D == 64 || D == 128) &&
         (a.bs == 16 || a.bs == 32) && tile_offsets_fit(a, D, a.head_group) &&
         (a.head_group == 1 || D == 64);
}

hipError_t launch_decode_streamk_plan_in(const DecodeArgs& a, int D, hipStream_t s) {
  if (!a.plan_in || !plan_handover_supported(a, D)) return hipErrorInvalidValue;
  if (D == 64) {
    if (a.head_group == 2)
      return a.bs == 16 ? launch_sk_plan_in<64, 16, 2>(a, s) : launch_sk_plan_in<64, 32, 2>(a, s);
    return a.bs == 16 ? launch_sk_plan_in<64, 16, 1>(a, s) : launch_sk_plan_in<64, 32, 1>(a, s);
  }
  return a.bs == 16 ? launch_sk_plan_in<128, 16, 1>(a, s) : launch_sk_plan_in<128, 32, 1>(a, s);
}

hipError_t launch_kv_write_plan(const DecodeArgs& a, const KVWriteArgs& w, bool vec,
                                hipStream_t s) {
  if (!a.plan_out || a.pair_per_wg || a.num_seqs > kSkMaxSeqs) return hipErrorInvalidValue;
  constexpr int NTHR = 64 * kSkWaves;
  const int per_row = vec ? w.D / 8 : w.D;
  const int64_t total = (int64_t)w.num_seqs * w.hkv * per_row;
  int64_t blocks = (total + NTHR - 1) / NTHR;
  if (blocks < 1) blocks = 1;
  if (blocks > 65535) blocks = 65535;
  if (vec)
    kv_write_plan_kernel<kSkWaves, true><<<(unsigned)blocks + 1, NTHR, 0, s>>>(a, w);
  else
    kv_write_plan_kernel<kSkWaves, false><<<(unsigned)blocks + 1, NTHR, 0, s>>>(a, w);
  return hipGetLastError();
}

// Kv heads a wavefront handles together for this shape.
hipError_t launch_decode_streamk(const DecodeArgs& a, int D, hipStream_t s) {
  if (a.plan_in) return launch_decode_streamk_plan_in(a, D, s);
  const int hg = a.head_group;
  if (hg != 1 && !(hg == 2 && D <= 64 && a.hkv % 2 == 0)) return hipErrorInvalidValue;
  switch (D) {
    case 32: return hg == 2 ? launch_sk_bs<32, 2>(a, s) : launch_sk_bs<32, 1>(a, s);
    case 64: return hg == 2 ? launch_sk_bs<64, 2>(a, s) : launch_sk_bs<64, 1>(a, s);
    case 128: return launch_sk_bs<128, 1>(a, s);
    case 256: return launch_sk_bs<256, 1>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace pa
