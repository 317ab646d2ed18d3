// Stream-K paged decode attention for gfx950 (MI355X).
//
// Schedule. The work is the list of (sequence, kv-head group) pairs, each a
// run of 16-token tiles; the list is ordered sequence-major. A persistent grid
// of G workgroups (two per CU, four wavefronts each) splits the concatenated
// tile list into G equal contiguous ranges, so every workgroup streams the
// same number of bytes however skewed the sequence lengths are. Every
// workgroup derives the plan itself: its threads load the lengths, scan the
// per-sequence tile counts into LDS and binary-search their range's first pair.
//
// Within a range the workgroup walks pair segments. The four wavefronts take
// the segment's chunks (NT tiles) round-robin, each keeping an online softmax
// per query head, and merge their states through LDS at the end of the
// segment. A pair wholly inside the range is written as final fp16 output; a
// pair cut by a range boundary leaves an fp32 partial record (at most two per
// workgroup) that merge_streamk_kernel combines by log-sum-exp.
//
// Per tile a wavefront loads the K and V rows of HG adjacent kv heads with
// whole-cache-line, non-temporal 16-byte loads (whole contiguous token rows
// when HG * head_dim * 2 bytes is the row), stages them through LDS, computes
// S^T = K Q^T on MFMA for the whole query group of each head (K read back in
// the MFMA operand layout), and O^T += V^T P^T on MFMA with V^T read back
// transposed (see pa_decode.hip for the operand layouts). Block ids are
// fetched two chunks ahead and K/V one chunk ahead of the computation.
#include "pa_common.h"

namespace pa {

namespace {

constexpr int kXcds = 8;  // accelerator complex dies of an MI355X, each with its own L2

__device__ inline f16x8 zero8() { return f16x8{0, 0, 0, 0, 0, 0, 0, 0}; }
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
__device__ inline f16x8 load_stream(const f16* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(p));
}

template <int BS>
__device__ inline int blk_of(int t, int bs) {
  if constexpr (BS > 0) return t / BS; else return t / bs;
}

template <int BS>
__device__ inline int off_of(int t, int bs) {
  if constexpr (BS > 0) return t % BS; else return t % bs;
}

}  // namespace

// First workgroup whose range contains tile x of a T-tile list split G ways.
__host__ __device__ inline int wg_of(int64_t x, int64_t T, int G) {
  return (int)(((x + 1) * G - 1) / T);
}

__host__ __device__ inline int64_t range_start(int w, int64_t T, int G) {
  return (int64_t)w * T / G;
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
  constexpr int NID = (BS > 0 && BS % 16 == 0) ? 1 : NI;  // block ids per tile per lane
  static_assert(NI * 64 == 16 * CPR, "tile must split into whole 64-lane loads");
  constexpr int VST = NT * HG * 16 * LS;  // halves of V staging per wavefront
  constexpr int CMB = HG * 16 * (D + 2);  // floats of merge state per wavefront
  // The merge state gets its own LDS when both fit two workgroups per CU; then
  // no barrier is needed after a merge (the next merge's entry barrier orders
  // it), so the merge's global stores never stall the wavefronts.
  constexpr bool SEPARATE = NW * (VST * 2 + CMB * 4) + 8 * kSkMaxSeqs + 64 <= 80 * 1024;
  constexpr int WAVE_BYTES = SEPARATE ? VST * 2 + CMB * 4 : (VST * 2 > CMB * 4 ? VST * 2 : CMB * 4);
  constexpr int CMB_OFF = SEPARATE ? VST * 2 : 0;  // byte offset of the merge state
  constexpr int PER = kSkMaxSeqs / NTHR;  // sequences planned per thread
  constexpr int REC = record_floats(D);
  static_assert(PER * NTHR == kSkMaxSeqs, "plan layout");

  __shared__ __attribute__((aligned(16))) char smem[NW * WAVE_BYTES];
  __shared__ int s_pref[kSkMaxSeqs + 1];
  __shared__ int s_len[kSkMaxSeqs];
  __shared__ int s_wtot[NW];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int row = lane & 15;
  const int grp = lane >> 4;
  const int B = a.num_seqs;
  const int NHG = a.hkv / HG;
  const int bs = BS > 0 ? BS : a.bs;
  const int G = gridDim.x;
  // Workgroup i is dispatched to XCD i % 8. Renumber so that each XCD owns a
  // contiguous run of ranges: neighbouring sequences (which is where shared
  // prefix blocks sit) then run on the same XCD and share its L2.
  const int wg = [&] {
    const int n8 = G / kXcds, rem = G % kXcds;
    const int xcd = blockIdx.x % kXcds, k = blockIdx.x / kXcds;
    return xcd * n8 + (xcd < rem ? xcd : rem) + k;
  }();

  // ---- plan: clamped lengths and the exclusive prefix of tiles per sequence ----
  {
    int cnt[PER];
    int local = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int b = tid * PER + i;
      int n = 0;
      if (b < B) {
        const int L = clamped_len(a, b);
        s_len[b] = L;
        n = (L + 15) >> 4;
      }
      cnt[i] = n;
      local += n;
    }
    int incl = local;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(incl, off);
      if (lane >= off) incl += y;
    }
    if (lane == 63) s_wtot[wave] = incl;
    __syncthreads();
    int run = incl - local;
    int total = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      if (w < wave) run += s_wtot[w];
      total += s_wtot[w];
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int b = tid * PER + i;
      if (b < B) s_pref[b] = run;
      run += cnt[i];
    }
    if (tid == 0) s_pref[B] = total;
    __syncthreads();
  }
  if (wg == 0 && a.pref) {
    for (int b = tid; b <= B; b += NTHR) a.pref[b] = s_pref[b];
  }

  // Zero-length sequences have no tiles; their rows are written as zeros.
  const int Hq = a.hkv * a.g;
  for (int b = wg; b < B; b += G) {
    if (s_pref[b + 1] == s_pref[b]) {
      for (int i = tid; i < Hq * D; i += NTHR) {
        const int hq = i / D;
        a.out[(int64_t)b * a.o_sb + (int64_t)hq * a.o_sh + (i - hq * D)] = (f16)0.f;
      }
    }
  }

  // Workgroups beyond the tile count get no range, so every range is non-empty.
  const int64_t T = (int64_t)NHG * s_pref[B];
  const int Ge = (int)(T < G ? T : G);
  if (wg >= Ge) return;
  const int64_t x0 = range_start(wg, T, Ge);
  const int64_t x1 = range_start(wg + 1, T, Ge);

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

  char* my_smem = smem + wave * WAVE_BYTES;
  f16* vst = reinterpret_cast<f16*>(my_smem);

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
    const int nt_b = s_pref[b + 1] - s_pref[b];
    const int64_t base = (int64_t)NHG * s_pref[b];
    const int hg0 = (int)((x - base) / nt_b);
    const int64_t pstart = base + (int64_t)hg0 * nt_b;
    const int64_t pend = pstart + nt_b;
    const int s0 = (int)(x - pstart);
    const int s1 = (int)((x1 < pend ? x1 : pend) - pstart);
    const bool first = s0 == 0;
    const bool last = pend <= x1;
    const int L = s_len[b];
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
          const int t = row_token(s0 + k * NT + nt, NID == 1 ? 0 : nat_row(j));
          ids[nt][j] = btrow[(int64_t)blk_of<BS>(t, bs) * a.bt_sk];
        }
    };
    auto load_kv = [&](int k, const int (&ids)[NT][NID], f16x8 (&kb)[NT][NI], f16x8 (&vb)[NT][NI]) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int ti = s0 + k * NT + nt;
        if (ti < s1) {
#pragma unroll
          for (int i = 0; i < NI; ++i) {
            const int t = row_token(ti, nat_row(i));
            const int64_t id = min(max(ids[nt][NID == 1 ? 0 : i], 0), a.num_blocks - 1);
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
    auto stage = [&](int k, f16x8 (&buf)[NT][NI], bool zero_tail) {
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
            const bool valid = !zero_tail || ti * 16 + r < L;
            *reinterpret_cast<f16x8*>(&vst[((nt * HG + hg) * 16 + r) * LS + d0]) =
                valid ? buf[nt][i] : zero8();
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

    auto compute = [&](int k, f16x8 (&kb)[NT][NI], f16x8 (&vb)[NT][NI]) {
      // K through LDS into the MFMA operand layout (lane: token row, 8-wide k slice).
      stage(k, kb, false);
      wave_lds_fence();
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
            const f16* kt = vst + ((nt * HG + hg) * 16 + row) * LS + grp * 8;
            f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NC; ++c)
              s = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const f16x8*>(kt + 32 * c),
                                                         qf[hg][c], s, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int tok = ti * 16 + grp * 4 + r;
              const float xv = tok < L ? s[r] * a.scale_log2 : kNegInf;
              xs[nt][hg][r] = xv;
              mloc[hg] = fmaxf(mloc[hg], xv);
            }
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) xs[nt][hg][r] = kNegInf;
          }
        }
      }
      wave_lds_fence();  // K reads are done before V takes the staging buffer
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
      // V rows to LDS (rows past the sequence end as zeros: 0 * garbage is never NaN).
      stage(k, vb, true);
      wave_lds_fence();
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
            const f16* vt = vst + (nt * HG + hg) * 16 * LS;
#pragma unroll
            for (int nd = 0; nd < ND; ++nd) {
              f16x4 av;
#pragma unroll
              for (int r = 0; r < 4; ++r) av[r] = vt[(grp * 4 + r) * LS + nd * 16 + row];
              acc[hg][nd] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, ph, acc[hg][nd], 0, 0, 0);
              acc[hg][nd] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, pl, acc[hg][nd], 0, 0, 0);
            }
          }
        }
      }
      wave_lds_fence();
    };

    const int nck = (s1 - s0 + NT - 1) / NT;
    int k = wave;
    if (k < nck) {
      f16x8 kb0[NT][NI], vb0[NT][NI], kb1[NT][NI], vb1[NT][NI];
      int idsA[NT][NID], idsB[NT][NID];
      load_ids(k, idsA);
      if (k + NW < nck) load_ids(k + NW, idsB);
      load_kv(k, idsA, kb0, vb0);
      for (; k < nck; k += 2 * NW) {
        if (k + 2 * NW < nck) load_ids(k + 2 * NW, idsA);
        if (k + NW < nck) load_kv(k + NW, idsB, kb1, vb1);
        compute(k, kb0, vb0);
        if (k + NW >= nck) break;
        if (k + 3 * NW < nck) load_ids(k + 3 * NW, idsB);
        if (k + 2 * NW < nck) load_kv(k + 2 * NW, idsA, kb0, vb0);
        compute(k + NW, kb1, vb1);
      }
    }

    // ---- merge the wavefronts' states through LDS ----
    float* cm = reinterpret_cast<float*>(my_smem + CMB_OFF);
    __syncthreads();  // V staging done (aliased case); the previous merge is read
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
        *reinterpret_cast<f32x4*>(&cm[2 * HG * 16 + (hg * 16 + row) * D + nd * 16 + grp * 4]) =
            acc[hg][nd];
    }
    __syncthreads();
    const int nout = HG * a.g * D;
    for (int i = tid; i < nout; i += NTHR) {
      const int hg = i / (a.g * D);
      const int rem = i - hg * a.g * D;
      const int hd = rem / D;
      const int d = rem - hd * D;
      float M = kNegInf;
#pragma unroll
      for (int w = 0; w < NW; ++w)
        M = fmaxf(M, reinterpret_cast<const float*>(smem + w * WAVE_BYTES + CMB_OFF)[hg * 16 + hd]);
      float num = 0.f, den = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float* c = reinterpret_cast<const float*>(smem + w * WAVE_BYTES + CMB_OFF);
        const float mw = c[hg * 16 + hd];
        const float sc = mw == kNegInf ? 0.f : fast_exp2(mw - M);
        den += sc * c[HG * 16 + hg * 16 + hd];
        num += sc * c[2 * HG * 16 + (hg * 16 + hd) * D + d];
      }
      if (first && last) {
        a.out[(int64_t)b * a.o_sb + (int64_t)((h0 + hg) * a.g + hd) * a.o_sh + d] =
            (f16)(den > 0.f ? num / den : 0.f);
      } else {
        float* rec = a.recs + ((int64_t)(wg * 2 + (first ? 1 : 0)) * HG + hg) * REC;
        if (d == 0) {
          rec[hd] = M;
          rec[16 + hd] = den;
        }
        rec[32 + hd * D + d] = num;
      }
    }
    if constexpr (!SEPARATE) __syncthreads();  // the merge state aliases V staging

    x = pend;
    if (x < x_end && x >= (int64_t)NHG * s_pref[b + 1]) {
      ++b;
      while (b < B - 1 && s_pref[b + 1] == s_pref[b]) ++b;
    }
  }
  }
}

// Combines the partial records of pairs cut by workgroup range boundaries.
// One workgroup per pair, one thread per output element. The pair's records
// are those of workgroups wa..wb (wa's tail slot, the others' head slots);
// they are read eight at a time with every load issued before any is used,
// and folded in with an online log-sum-exp.
template <int D, int HG>
__global__ __launch_bounds__(1024) void merge_streamk_kernel(DecodeArgs a) {
  constexpr int REC = record_floats(D);
  constexpr int BATCH = 8;
  const int NHG = a.hkv / HG;
  const int p = blockIdx.x;
  const int b = p / NHG;
  const int hgp = p - b * NHG;
  const int sb = a.pref[b];
  const int nt = a.pref[b + 1] - sb;
  if (nt == 0) return;
  const int64_t T = (int64_t)NHG * a.pref[a.num_seqs];
  const int G = (int)(T < a.num_wg ? T : a.num_wg);
  const int64_t pstart = (int64_t)NHG * sb + (int64_t)hgp * nt;
  const int wa = wg_of(pstart, T, G);
  const int wb = wg_of(pstart + nt - 1, T, G);
  if (wa == wb) return;
  const int nrec = wb - wa + 1;
  const int nout = HG * a.g * D;
  for (int i = threadIdx.x; i < nout; i += blockDim.x) {
    const int hg = i / (a.g * D);
    const int rem = i - hg * a.g * D;
    const int hd = rem / D;
    const int d = rem - hd * D;
    float M = kNegInf, num = 0.f, den = 0.f;
    for (int k0 = 0; k0 < nrec; k0 += BATCH) {
      float mv[BATCH], lv[BATCH], av[BATCH];
#pragma unroll
      for (int j = 0; j < BATCH; ++j) {
        const int k = k0 + j;
        const int kk = k < nrec ? k : 0;
        const int slot = 2 * (wa + kk) + (kk == 0 ? 1 : 0);
        const float* r = a.recs + ((int64_t)slot * HG + hg) * REC;
        mv[j] = r[hd];
        lv[j] = r[16 + hd];
        av[j] = r[32 + hd * D + d];
        if (k >= nrec) mv[j] = kNegInf;
      }
      float mb = M;
#pragma unroll
      for (int j = 0; j < BATCH; ++j) mb = fmaxf(mb, mv[j]);
      const float sc = M == kNegInf ? 0.f : fast_exp2(M - mb);
      num *= sc;
      den *= sc;
#pragma unroll
      for (int j = 0; j < BATCH; ++j) {
        const float w = mv[j] == kNegInf ? 0.f : fast_exp2(mv[j] - mb);
        num += w * av[j];
        den += w * lv[j];
      }
      M = mb;
    }
    a.out[(int64_t)b * a.o_sb + (int64_t)((hgp * HG + hg) * a.g + hd) * a.o_sh + d] =
        (f16)(den > 0.f ? num / den : 0.f);
  }
}

// ---------------------------------------------------------------------------
// Launchers.
// ---------------------------------------------------------------------------
namespace {

constexpr int kSkWaves = 4;

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
  const int pairs = a.num_seqs * (a.hkv / HG);
  if (pairs > 0) merge_streamk_kernel<D, HG><<<pairs, 1024, 0, s>>>(a);
  return hipGetLastError();
}

template <int D, int HG>
hipError_t launch_sk_bs(const DecodeArgs& a, hipStream_t s) {
  switch (a.bs) {
    case 8: return launch_sk<D, 8, HG>(a, s);
    case 16: return launch_sk<D, 16, HG>(a, s);
    case 32: return launch_sk<D, 32, HG>(a, s);
    default: return launch_sk<D, 0, HG>(a, s);
  }
}

}  // namespace

// Kv heads a wavefront handles together for this shape.
int streamk_head_group(int num_kv_heads, int D) {
  return (D <= 64 && num_kv_heads % 2 == 0) ? 2 : 1;
}

hipError_t launch_decode_streamk(const DecodeArgs& a, int D, hipStream_t s) {
  const int hg = streamk_head_group(a.hkv, D);
  switch (D) {
    case 32: return hg == 2 ? launch_sk_bs<32, 2>(a, s) : launch_sk_bs<32, 1>(a, s);
    case 64: return hg == 2 ? launch_sk_bs<64, 2>(a, s) : launch_sk_bs<64, 1>(a, s);
    case 128: return launch_sk_bs<128, 1>(a, s);
    case 256: return launch_sk_bs<256, 1>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace pa
