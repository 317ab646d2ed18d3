// Stream-K paged decode attention for gfx950 (MI355X).
//
// Schedule. The work is the list of (sequence, kv-head group) pairs, each a
// run of 16-token tiles; the list is ordered sequence-major. A persistent grid
// of G workgroups (one per CU, eight wavefronts each) splits the concatenated
// tile list into G equal contiguous ranges, so every workgroup streams the
// same number of bytes however skewed the sequence lengths are. Every
// workgroup derives the plan itself: its threads load the lengths, scan the
// per-sequence tile counts into LDS and binary-search their range's first pair.
//
// Within a range the workgroup walks pair segments. Wavefront w takes chunks
// (NT tiles) w, w + 8, w + 16, ... of the segment, keeping an online softmax
// per query head, and the eight wavefronts merge their states through LDS in
// a fixed order at the end of the segment, so results are the same bits on
// every run. A pair wholly inside the range is written as final fp16 output;
// a pair cut by a range boundary leaves an fp32 partial record (at most two
// per workgroup), and the last workgroup to count an arrival for such a pair
// combines its records by log-sum-exp, in record order.
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

// First workgroup whose range contains tile x of a T-tile list split G ways.
__host__ __device__ inline int wg_of(int64_t x, int64_t T, int G) {
  return (int)(((x + 1) * G - 1) / T);
}

__host__ __device__ inline int64_t range_start(int w, int64_t T, int G) {
  return (int64_t)w * T / G;
}

// Exclusive prefix sums over a workgroup of NW wavefronts, PER values per
// thread (thread t holds entries t * PER .. t * PER + PER - 1); returns the
// total. s_tot holds NW ints; the call starts and ends with a barrier.
template <int PER, int NW>
__device__ inline int block_excl_sum(int (&v)[PER], int* s_tot, int lane, int wave) {
  int local = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) local += v[i];
  int incl = local;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off);
    if (lane >= off) incl += y;
  }
  __syncthreads();
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
  __syncthreads();
  return total;
}

template <int D, int NT, int BS, int HG, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2)))
void decode_streamk_kernel(DecodeArgs a) {
  constexpr int NC = D / 32;
  constexpr int ND = D / 16;
  constexpr int LS = D + 8;
  constexpr int NTHR = 64 * NW;
  constexpr int CPR = HG * D / 8;          // 16-byte chunks per token row of a head group
  constexpr int NI = 16 * CPR / 64;        // load instructions per tile, for K and for V
  // A 16-token tile lies inside one block when 16 divides the block size: its
  // block id and row base are then wavefront-uniform.
  constexpr bool UNIFORM_TILE = BS > 0 && BS % 16 == 0;
  constexpr int NID = UNIFORM_TILE ? 1 : NI;  // block ids per tile per lane
  constexpr int RS = 64 / CPR;                // token rows one load instruction covers
  static_assert(NI * 64 == 16 * CPR, "tile must split into whole 64-lane loads");
  static_assert(RS * CPR == 64, "a load instruction must cover whole rows");
  constexpr int VST = NT * HG * 16 * LS;  // halves of one staging buffer (K or V) per wavefront
  constexpr int CMB = 32 * HG + HG * ND * 64 * 4;  // floats of merge state per wavefront
  // Per wavefront: a K and a V staging buffer; the merge state reuses the same
  // bytes at segment ends.
  constexpr int WAVE_BYTES = (2 * VST * 2 > CMB * 4 ? 2 * VST * 2 : CMB * 4);
  constexpr int PER = kSkMaxSeqs / NTHR;  // sequences planned per thread
  constexpr int REC = record_floats(D);
  static_assert(PER * NTHR == kSkMaxSeqs, "plan layout");
  __shared__ __attribute__((aligned(16))) char smem[NW * WAVE_BYTES];
  __shared__ int s_pref[kSkMaxSeqs + 1];  // sequence -> first tile position (per kv-head group)
  __shared__ int s_wtot[NW];
  __shared__ int s_nmerge;                // pairs listed for merging
  __shared__ int s_mlist[NTHR];           // pairs whose records this workgroup completed

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int row = lane & 15;
  const int grp = lane >> 4;
  const int B = a.num_seqs;
  const int NHG = a.hkv / HG;
  const int bs = BS > 0 ? BS : a.bs;
  const int G = gridDim.x;

  // ---- plan: clamped lengths and the exclusive prefix of tiles per sequence ----
  {
    int cnt[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int b = tid * PER + i;
      const int n = b < B ? (clamped_len(a, b) + 15) >> 4 : 0;
      cnt[i] = n > 0 ? n + a.seg_cost : 0;  // pair width: its tiles plus the segment overhead
    }
    const int total = block_excl_sum<PER, NW>(cnt, s_wtot, lane, wave);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int b = tid * PER + i;
      if (b < B) s_pref[b] = cnt[i];
    }
    if (tid == 0) s_pref[B] = total;
    __syncthreads();
  }

  // Zero-length sequences have no tiles; their rows are written as zeros.
  const int Hq = a.hkv * a.g;
  for (int b = blockIdx.x; b < B; b += G) {
    if (s_pref[b + 1] == s_pref[b]) {
      for (int i = tid; i < Hq * D; i += NTHR) {
        const int hq = i / D;
        a.out[(int64_t)b * a.o_sb + (int64_t)hq * a.o_sh + (i - hq * D)] = (f16)0.f;
      }
    }
  }

  // Ranges: at least min_range tile positions each, at most one per
  // workgroup; workgroups beyond them get no range.
  const int64_t T = (int64_t)NHG * s_pref[B];
  const int64_t Gw = (T + a.min_range - 1) / a.min_range;
  const int Ge = (int)(Gw < G ? Gw : G);  // 0 when every sequence is empty

  // The first A workgroups take part. Workgroup i is dispatched to XCD i % 8;
  // renumber the A of them so that each XCD owns a contiguous run of ranges
  // (or pairs): neighbouring sequences, which is where shared prefix blocks
  // sit, then run on the same XCD and share its L2, and every XCD gets work
  // when A < G.
  const int A = a.pair_per_wg ? (B * NHG < G ? B * NHG : G) : Ge;
  if ((int)blockIdx.x >= A) return;
  const int wg = [&] {
    const int n8 = A / kXcds, rem = A % kXcds;
    const int xcd = blockIdx.x % kXcds, k = blockIdx.x / kXcds;
    return xcd * n8 + (xcd < rem ? xcd : rem) + k;
  }();
  int64_t x0, x1;
  if (a.pair_per_wg) {
    // Small batches of short pairs: workgroup w takes pair w whole, so no pair
    // is cut, no partial record is written and no merge is needed.
    const int pb = wg / NHG;
    const int width = s_pref[pb + 1] - s_pref[pb];
    if (width == 0) return;  // a zero-length sequence: its rows were written above
    x0 = (int64_t)NHG * s_pref[pb] + (int64_t)(wg - pb * NHG) * width;
    x1 = x0 + width;
  } else {
    x0 = range_start(wg, T, Ge);
    x1 = range_start(wg + 1, T, Ge);
  }

  // First pair: the last sequence whose pairs start at or before x0.
  int b;
  {
    int lo = 0, hi = B - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if ((int64_t)NHG * s_pref[mid] <= x0) lo = mid; else hi = mid - 1;
    }
    b = lo;
  }

  // Byte offset of this lane's 16-byte piece within a tile, relative to the
  // tile's first row at the group's first kv head (same for every tile).
  uint32_t k_lane = 0, v_lane = 0;
  if constexpr (UNIFORM_TILE) {
    const int lrow = lane / CPR, lcol = (lane % CPR) * 8;
    const int lhg = lcol / D, ld0 = lcol - lhg * D;
    k_lane = (uint32_t)(2 * (lrow * a.k_st + lhg * a.k_sh + ld0));
    v_lane = (uint32_t)(2 * (lrow * a.v_st + lhg * a.v_sh + ld0));
  }
  char* my_smem = smem + wave * WAVE_BYTES;
  f16* kst = reinterpret_cast<f16*>(my_smem);  // K staging
  f16* vst = kst + VST;                          // V staging

  // Partial records, two per range: slot 2 w + 1 for the pair range w cuts at
  // its end, slot 2 w for the pair it continues from earlier ranges.
  const auto rec_rsrc = tile_rsrc(a.recs, a.recs_bytes);

  // The ranges wa .. wa + nrec - 1 a cut pair spans.
  auto pair_span = [&](int p, int& wa, int& nrec) {
    const int pb = p / NHG;
    const int nt = s_pref[pb + 1] - s_pref[pb] - a.seg_cost;
    const int64_t ps = (int64_t)NHG * s_pref[pb] + (int64_t)(p - pb * NHG) * (nt + a.seg_cost) + a.seg_cost;
    wa = wg_of(ps, T, Ge);
    nrec = wg_of(ps + nt - 1, T, Ge) - wa + 1;
  };

  // Arrivals this workgroup has counted and not yet resolved: thread t < npend
  // counted one for pair s_mlist[t] and holds the value its counter increment
  // returned.
  int npend = 0;
  int my_old = 0;

  // Resolves the counted arrivals: a pair whose count this workgroup completed
  // is merged here -- its records in range order, by an online log-sum-exp over
  // 16-byte device-coherent loads (each thread four accumulators of one query
  // head, eight records in flight), all such pairs of the workgroup at once --
  // and its counter is reset to zero for the next launch.
  auto resolve = [&]() {
    const int my_pair = tid < npend ? s_mlist[tid] : 0;
    if (tid == 0) s_nmerge = 0;
    __syncthreads();
    if (tid < npend) {
      int wa, nrec;
      pair_span(my_pair, wa, nrec);
      if (my_old == nrec - 1) s_mlist[atomicAdd(&s_nmerge, 1)] = my_pair;
    }
    __syncthreads();
    const int nmg = s_nmerge;
    constexpr int DQ = D / 4;
    const int per = HG * a.g * DQ;
    for (int it = tid; it < nmg * per; it += NTHR) {
      const int e = it / per;
      int rem = it - e * per;
      const int hh = rem / (a.g * DQ);
      rem -= hh * a.g * DQ;
      const int qr = rem / DQ;
      const int dq = rem - qr * DQ;
      const int p = s_mlist[e];
      int wa, n;
      pair_span(p, wa, n);
      float M = kNegInf, den = 0.f;
      f32x4 num = {0.f, 0.f, 0.f, 0.f};
      for (int k0 = 0; k0 < n; k0 += 8) {
        float mv[8], lv[8];
        f32x4 av[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int kk = k0 + k < n ? k0 + k : 0;
          const int slot = 2 * (wa + kk) + (kk == 0 ? 1 : 0);
          const int base = (slot * HG + hh) * REC;
          mv[k] = load_coherent4(rec_rsrc, 4 * (base + qr));
          lv[k] = load_coherent4(rec_rsrc, 4 * (base + 16 + qr));
          av[k] = load_coherent16(rec_rsrc, 4 * (base + 32 + qr * D + dq * 4));
          if (k0 + k >= n) mv[k] = kNegInf;
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
      const int pb = p / NHG, hgp = p - pb * NHG;
      *reinterpret_cast<f16x4*>(a.out + (int64_t)pb * a.o_sb +
                                (int64_t)((hgp * HG + hh) * a.g + qr) * a.o_sh + dq * 4) = ov;
    }
    for (int e = tid; e < nmg; e += NTHR)
      __hip_atomic_store(a.cnt + s_mlist[e], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    npend = 0;
  };


  // Segment order: a range starts with at most one segment that continues a
  // pair begun in an earlier range. It is processed last, so every workgroup
  // starts on the first tiles of a pair: the leading blocks of all sequences
  // -- where sequences share prefix blocks -- are read close together in time
  // and repeated reads of a shared block find it in the L2 / MALL.
  int64_t cont_end = x0;  // end of the leading continuation segment (x0 if none)
  {
    const int64_t base0 = (int64_t)NHG * s_pref[b];
    const int nt0 = s_pref[b + 1] - s_pref[b];
    const int64_t ps0 = base0 + (x0 - base0) / nt0 * nt0;
    if (ps0 < x0) cont_end = ps0 + nt0 < x1 ? ps0 + nt0 : x1;
  }
  const int b_cont = b;
  if (cont_end > x0 && cont_end < x1 && cont_end >= (int64_t)NHG * s_pref[b + 1]) {
    ++b;
    while (b < B - 1 && s_pref[b + 1] == s_pref[b]) ++b;
  }

  for (int pass = 0; pass < 2; ++pass) {
  int64_t x = pass == 0 ? cont_end : x0;
  const int64_t x_end = pass == 0 ? x1 : cont_end;
  if (pass == 1) b = b_cont;
  while (x < x_end) {
    const int nt_b = s_pref[b + 1] - s_pref[b];  // pair width, seg_cost included
    const int64_t base = (int64_t)NHG * s_pref[b];
    const int hg0 = (int)((x - base) / nt_b);
    const int64_t pstart = base + (int64_t)hg0 * nt_b;
    const int64_t pend = pstart + nt_b;
    // Segment bounds in real tiles (the pair's first seg_cost positions stand
    // for its fixed overhead and hold no tiles), wavefront-uniform by
    // construction; readfirstlane makes that visible to the compiler, so the
    // loop below keeps uniform branches (a branch it must treat as divergent
    // gets restructured into paths that skip loads, which spoils the wait
    // counts of the load pipeline).
    const int s0 = __builtin_amdgcn_readfirstlane(max((int)(x - pstart) - a.seg_cost, 0));
    const int s1 = __builtin_amdgcn_readfirstlane(
        max((int)((x1 < pend ? x1 : pend) - pstart) - a.seg_cost, 0));
    const bool first = s0 == 0;
    const bool last = pend <= x1;
    if (s1 > s0) {  // else the range holds only overhead positions of this pair
      const int L = __builtin_amdgcn_readfirstlane(clamped_len(a, b));
      const int h0 = hg0 * HG;  // first kv head of the group

      // ---- this wavefront's share of the segment ----
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
      const int32_t* btrow = a.bt + (int64_t)b * a.bt_sb;
      const int tok_fallback = s0 * 16;  // a valid token of this segment

      // Natural-layout loads: instruction i of a tile gives lane l the 16-byte
      // chunk f = 64 i + l of the tile's 16 rows x (HG * D) halves, i.e. row
      // f / CPR, halves (f % CPR) * 8 of the row's head-group slice. Each
      // instruction thus reads whole row slices (whole cache lines).
      auto nat_row = [&](int i) { return (64 * i + lane) / CPR; };
      auto nat_col = [&](int i) { return ((64 * i + lane) % CPR) * 8; };
      auto row_token = [&](int ti, int r) {
        const int t = ti * 16 + r;
        return (ti < s1 && t < L) ? t : tok_fallback;
      };
      auto load_ids = [&](int k, int (&ids)[NT][NID]) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
          for (int j = 0; j < NID; ++j) {
            // A uniform tile lies in one block; otherwise each lane looks up the
            // block of its own row (also when one instruction covers the tile).
            const int t = row_token(s0 + k * NT + nt, UNIFORM_TILE ? 0 : nat_row(j));
            if constexpr (UNIFORM_TILE)
              ids[nt][j] = load_uniform(btrow + (int64_t)blk_of<BS>(t, bs) * a.bt_sk);
            else
              ids[nt][j] = btrow[(int64_t)blk_of<BS>(t, bs) * a.bt_sk];
          }
      };
      auto load_kv = [&](int k, const int (&ids)[NT][NID], u32x4 (&kb)[NT][NI], u32x4 (&vb)[NT][NI]) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int ti = s0 + k * NT + nt;
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
      auto stage = [&](int k, u32x4 (&buf)[NT][NI], f16* dst, bool zero_tail) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int ti = s0 + k * NT + nt;
          if (ti < s1) {
#pragma unroll
            for (int i = 0; i < NI; ++i) {
              const int r = nat_row(i);
              const int col = nat_col(i);
              const int hg = col / D;
              const int d0 = col - hg * D;
              *reinterpret_cast<u32x4*>(&dst[((nt * HG + hg) * 16 + r) * LS + d0]) = buf[nt][i];
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
                  *reinterpret_cast<f16x8*>(&dst[((nt * HG + hg) * 16 + r) * LS + d0]) = zero8();
              }
            }
          }
        }
      };

      float m_run[HG], l_run[HG];
      f32x4 acc[HG][ND];
#pragma unroll
      for (int hg = 0; hg < HG; ++hg) {
        m_run[hg] = kNegInf;
        l_run[hg] = 0.f;
#pragma unroll
        for (int i = 0; i < ND; ++i) acc[hg][i] = f32x4{0.f, 0.f, 0.f, 0.f};
      }

      // Both K and V of chunk k go to LDS first, which frees their registers for
      // the loads of the chunk two steps ahead; the math then reads LDS only.
      auto stage_both = [&](int k, u32x4 (&kb)[NT][NI], u32x4 (&vb)[NT][NI]) {
        stage(k, kb, kst, false);
        stage(k, vb, vst, true);  // V rows past the sequence end as zeros: 0 * garbage is never NaN
        wave_lds_fence();
      };
      auto compute = [&](int k) {
        float xs[NT][HG][4];
        float mloc[HG];
#pragma unroll
        for (int hg = 0; hg < HG; ++hg) mloc[hg] = kNegInf;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int ti = s0 + k * NT + nt;
#pragma unroll
          for (int hg = 0; hg < HG; ++hg) {
            if (ti < s1) {
              const f16* kt = kst + ((nt * HG + hg) * 16 + row) * LS + grp * 8;
              f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
              for (int c = 0; c < NC; ++c)
                s = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const f16x8*>(kt + 32 * c),
                                                           qf[hg][c], s, 0, 0, 0);
              if (ti * 16 + 16 <= L) {  // wavefront-uniform: only the last tile is partial
#pragma unroll
                for (int r = 0; r < 4; ++r) xs[nt][hg][r] = s[r] * a.scale_log2;
              } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                  xs[nt][hg][r] = ti * 16 + grp * 4 + r < L ? s[r] * a.scale_log2 : kNegInf;
              }
#pragma unroll
              for (int r = 0; r < 4; ++r) mloc[hg] = fmaxf(mloc[hg], xs[nt][hg][r]);
            } else {
#pragma unroll
              for (int r = 0; r < 4; ++r) xs[nt][hg][r] = kNegInf;
            }
          }
        }
#pragma unroll
        for (int hg = 0; hg < HG; ++hg) {
          float m = mloc[hg];
          m = fmaxf(m, __shfl_xor(m, 16));
          m = fmaxf(m, __shfl_xor(m, 32));
          const float m_new = fmaxf(m_run[hg], m);
          const float alpha = fast_exp2(m_run[hg] - m_new);
          l_run[hg] *= alpha;
#pragma unroll
          for (int i = 0; i < ND; ++i) acc[hg][i] *= alpha;
          m_run[hg] = m_new;
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int ti = s0 + k * NT + nt;
          if (ti < s1) {
#pragma unroll
            for (int hg = 0; hg < HG; ++hg) {
              f16x4 ph, pl;
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const float pr = fast_exp2(xs[nt][hg][r] - m_run[hg]);
                l_run[hg] += pr;
                const f16 hi = (f16)pr;
                ph[r] = hi;
                pl[r] = (f16)(pr - (float)hi);
              }
              // V^T operand: lane (row, grp) needs V[4 grp + r][16 nd + row], r = 0..3,
              // which one transposing read of rows 4 grp..4 grp+3 delivers.
              const f16* vt = vst + ((nt * HG + hg) * 16 + grp * 4 + (row >> 2)) * LS + (row & 3) * 4;
#pragma unroll
              for (int nd = 0; nd < ND; ++nd) {
                const f16x4 av = lds_read_tr16(vt + nd * 16);
                acc[hg][nd] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, ph, acc[hg][nd], 0, 0, 0);
                acc[hg][nd] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, pl, acc[hg][nd], 0, 0, 0);
              }
            }
          }
        }
        wave_lds_fence();
      };

      // Wavefront-local pipeline over this wavefront's chunks: wavefront w
      // takes chunks w, w + NW, w + 2 NW, ... A fixed assignment (rather than
      // claims from a shared counter, which let faster wavefronts take more
      // chunks) keeps the summation order, and so the result bits, the same
      // on every run; it costs about 1% at large batches. Step s computes chunk c_s: K/V register sets Y0/Y1 hold steps s and
      // s+1, id sets X0/X1 the block ids of steps s+2 and s+3. At step s: stage
      // Y[s%2] into LDS, reuse it for the loads of step s+2 (ids in X[s%2]),
      // claim step s+3 and fetch its ids into X[(s+1)%2], then compute step s.
      // Claims are increasing per wavefront, so the first claim past the end
      // ends its work; loads of such chunks are issued anyway (empty resources,
      // clamped table reads) so that no branch separates them.
      const int nck = __builtin_amdgcn_readfirstlane((s1 - s0 + NT - 1) / NT);
      int next_chunk = wave;
      auto claim = [&]() {
        const int c = next_chunk;
        next_chunk += NW;
        return c;
      };
      {
        u32x4 kb0[NT][NI], vb0[NT][NI], kb1[NT][NI], vb1[NT][NI];
        int ids0[NT][NID], ids1[NT][NID];
        int c0 = claim();
        int c1 = claim();
        int c2 = claim();
        load_ids(c0, ids0);
        load_ids(c1, ids1);
        // The scheduler must keep the loads of step 0 ahead of those of step 1:
        // the loop's waits count on the older buffer being the one staged first.
        load_kv(c0, ids0, kb0, vb0);
        __builtin_amdgcn_sched_barrier(0);
        load_kv(c1, ids1, kb1, vb1);
        __builtin_amdgcn_sched_barrier(0);
        load_ids(c2, ids0);
        // Two steps per trip, one exit: both steps issue their loads on every
        // trip and only the LDS staging and the math of a step past the end are
        // skipped, so every path through the loop issues the same loads.
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

      // ---- merge the wavefronts' states through LDS ----
      // Every wavefront stores its maxima and denominators per head and its
      // accumulators in register layout (chunk j = hg * ND + nd: one f32x4 per
      // lane, so the 16-byte LDS writes are conflict-free). Wavefront w then
      // combines chunks j = w, w + NW, ... of all wavefronts and stores them.
      float* cm = reinterpret_cast<float*>(my_smem);
      __syncthreads();  // every wavefront is done with its staging buffers
#pragma unroll
      for (int hg = 0; hg < HG; ++hg) {
        float l = l_run[hg];
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        if (grp == 0) {
          cm[hg * 16 + row] = m_run[hg];
          cm[HG * 16 + hg * 16 + row] = l;
        }
#pragma unroll
        for (int nd = 0; nd < ND; ++nd)
          *reinterpret_cast<f32x4*>(&cm[32 * HG + ((hg * ND + nd) * 64 + lane) * 4]) = acc[hg][nd];
      }
      __syncthreads();
      for (int j = wave; j < HG * ND; j += NW) {
        const int hg = j / ND;
        const int nd = j - hg * ND;
        float mw[NW];
        float M = kNegInf;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          mw[w] = reinterpret_cast<const float*>(smem + w * WAVE_BYTES)[hg * 16 + row];
          M = fmaxf(M, mw[w]);
        }
        float den = 0.f;
        f32x4 num = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          const float* c = reinterpret_cast<const float*>(smem + w * WAVE_BYTES);
          const float sc = mw[w] == kNegInf ? 0.f : fast_exp2(mw[w] - M);
          den += sc * c[HG * 16 + hg * 16 + row];
          num += sc * *reinterpret_cast<const f32x4*>(&c[32 * HG + (j * 64 + lane) * 4]);
        }
        if (row < a.g) {
          if (first && last) {
            const float inv = den > 0.f ? 1.f / den : 0.f;
            f16x4 o;
#pragma unroll
            for (int r = 0; r < 4; ++r) o[r] = (f16)(num[r] * inv);
            *reinterpret_cast<f16x4*>(a.out + (int64_t)b * a.o_sb +
                                      (int64_t)((h0 + hg) * a.g + row) * a.o_sh + nd * 16 + grp * 4) = o;
          } else {
            const int rb = ((wg * 2 + (first ? 1 : 0)) * HG + hg) * REC;
            if (grp == 0 && nd == 0) {
              store_coherent(a.recs + rb + row, M);
              store_coherent(a.recs + rb + 16 + row, den);
            }
            store_coherent16(rec_rsrc, 4 * (rb + 32 + row * D + nd * 16 + grp * 4), num);
          }
        }
      }
      if (!(first && last)) {
        // Publish the record: every thread waits for its coherent stores to
        // complete, then one arrival is counted for the pair. The returned
        // count is only needed when the workgroup resolves its arrivals, so
        // the atomic's latency overlaps the rest of the range.
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == npend) {
          s_mlist[tid] = b * NHG + hg0;
          my_old = __hip_atomic_fetch_add(a.cnt + b * NHG + hg0, 1, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
        }
        ++npend;
      }
      __syncthreads();  // the merge state aliases the staging buffers of the next segment
    }
    x = pend;
    if (x < x_end && x >= (int64_t)NHG * s_pref[b + 1]) {
      ++b;
      while (b < B - 1 && s_pref[b + 1] == s_pref[b]) ++b;
    }
  }
  }

  // ---- pairs cut by range boundaries: the last workgroup to arrive merges ----
  // A pair spanning ranges wa..wb has one record per range (wa's tail slot,
  // the others' head slots); the workgroup whose arrival completes the count
  // combines them. A range cuts at most two pairs, so at most two arrivals
  // are pending here.
  resolve();
}

// ---------------------------------------------------------------------------
// Launchers.
// ---------------------------------------------------------------------------
namespace {

constexpr int kSkWaves = 8;

// Tiles per chunk: two chunks of K/V (one computing, one in flight) must fit
// the 256 VGPRs a wavefront has at two wavefronts per SIMD.
template <int D>
constexpr int sk_chunk_tiles(int hg) {
  return D <= 32 ? (hg == 2 ? 2 : 4) : (D <= 128 ? 2 : 1);
}

template <int D, int BS, int HG>
hipError_t launch_sk(const DecodeArgs& a, hipStream_t s) {
  constexpr int NT = sk_chunk_tiles<D>(HG);
  decode_streamk_kernel<D, NT, BS, HG, kSkWaves><<<a.num_wg, 64 * kSkWaves, 0, s>>>(a);
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

// Kv heads a wavefront handles together for this shape.
hipError_t launch_decode_streamk(const DecodeArgs& a, int D, hipStream_t s) {
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
