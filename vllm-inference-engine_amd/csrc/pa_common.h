// Shared definitions for the gfx950 paged-attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pa {

typedef _Float16 f16;
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kLog2e = 1.4426950408889634f;

// Physical block ids of one split are staged in LDS; this bounds the split length.
constexpr int kMaxIds = 512;

// Host-side error reporting (thread-local message read by pa_last_error()).
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// Argument bundle of the decode kernels. Element strides; head_dim stride is 1.
struct DecodeArgs {
  const f16* q;
  int64_t q_sb, q_sh;
  const f16* k;
  int64_t k_sb, k_st, k_sh;
  const f16* v;
  int64_t v_sb, v_st, v_sh;
  const int32_t* bt;  // block table rows
  int64_t bt_sb, bt_sk;
  const int32_t* lens;  // per-sequence lengths, or null: use uniform_len
  int uniform_len;
  f16* out;
  int64_t o_sb, o_sh;
  float* ws;  // split-K partial records, or v1 score rows
  int hkv, g, bs, num_blocks, max_blocks;
  int split_tiles, max_splits;
  int lpad;  // v1: padded score-row length
  float scale_log2;  // softmax scale times log2(e): scores live in the exp2 domain
  // Stream-K schedule (decode_streamk_kernel).
  int num_seqs;  // sequences in the batch
  int num_wg;    // workgroups of the persistent grid
  float* recs;   // 2 partial records per workgroup
  int* cnt;      // per-pair arrival counters, zero between launches
  // Fixed cost of a pair segment (pipeline fill, cross-wavefront merge),
  // in tiles: the schedule splits tiles plus this cost per pair evenly.
  int seg_cost;
  // Nonzero: one workgroup per (sequence, kv-head group) pair instead of
  // equal ranges of the pair list (small batches of short sequences).
  int pair_per_wg;
  int recs_bytes;  // size of the record area at recs
  // Stream-K ranges get at least this many tile positions each: a launch with
  // little work uses fewer ranges than workgroups (the rest exit at once).
  int min_range;
  int head_group;  // kv heads per stream-K pair (1 or 2)
  // Shared prefixes (block size a multiple of 16, head_dim <= 64): nonzero
  // lets the kernel find runs of neighbouring sequences whose leading table
  // entries are the same physical blocks and read those blocks once per run.
  int share;
  int max_members;  // sequences per sharing group (at most kPfxMaxMembers)
  int slot_recs;    // records per partial-record slot: max(head_group, kPfxColBlocks) when sharing
  // The stream-K plan (positions, then sharing information; layout of the
  // workspace head) computed by the K/V write launch just before this one on
  // the same stream, or null: every workgroup derives it.
  const int* plan_in;
  int* plan_out;  // where a K/V write launch leaves the plan
};

// Shared-prefix groups: leading table entries compared per sequence, most
// sequences per group, and column blocks of 16 query rows a prefix item's
// wavefront computes (the group's members times the query group size).
constexpr int kPfxCapBlocks = 64;
constexpr int kPfxMaxMembers = 8;
constexpr int kPfxColBlocks = 4;

// Members a sharing group may have at query group size g: whole members per
// 16-column block times the column blocks, at most kPfxMaxMembers.
__host__ __device__ constexpr int pfx_members(int g) {
  return (16 / g) * kPfxColBlocks < kPfxMaxMembers ? (16 / g) * kPfxColBlocks : kPfxMaxMembers;
}

// Stream-K limits: sequences whose tile prefix fits the LDS plan, the largest
// persistent grid the workspace is sized for, and the (sequence, kv-head
// group) pairs the counter region at the start of the workspace holds.
constexpr int kSkMaxSeqs = 1024;
constexpr int kSkMaxWG = 1024;
constexpr int kSkMaxPairs = 65536;
// Head of a stream-K workspace, ahead of the partial records: the pair
// counters (zero between launches), then the plan a K/V write launch leaves
// for the attention launch after it (each sequence's first list position,
// kSkMaxSeqs + 1 ints, then its sharing information, kSkMaxSeqs ints).
constexpr size_t kSkPairCounterBytes = (size_t)kSkMaxPairs * sizeof(int);
constexpr size_t kSkPlanBytes = (size_t)(2 * kSkMaxSeqs + 64) * sizeof(int);
constexpr size_t kSkCounterBytes = kSkPairCounterBytes + kSkPlanBytes;
// Persistent workgroups per compute unit (each of eight wavefronts).
constexpr int kSkWgPerCu = 1;

// Argument bundle of the K/V write kernel. Element strides; the sources may be
// arbitrary views, the caches have unit head_dim stride.
struct KVWriteArgs {
  const uint16_t* key;
  int64_t ks_b, ks_h, ks_d;
  const uint16_t* val;
  int64_t vs_b, vs_h, vs_d;
  uint16_t* kc;
  int64_t kc_sb, kc_st, kc_sh;
  uint16_t* vc;
  int64_t vc_sb, vc_st, vc_sh;
  const int32_t* bt;
  int64_t bt_sb, bt_sk;
  const int32_t* lens;  // per-sequence lengths, or null: use uniform_len
  int uniform_len;
  int num_seqs, hkv, D, bs, num_blocks, max_blocks;
};

// The K/V write's copies, items i0, i0 + step, ... of the num_seqs x hkv x
// (D / 8 or D) list: sequence b's new key and value rows go to the slot of
// position L - 1 (L = lens[b]), as 16-bit patterns (no float conversion), 16
// bytes per item with VEC, one element otherwise. Sequences with no tokens,
// a slot past the table or an out-of-range block id write nothing.
template <bool VEC>
__device__ inline void kv_write_rows(const KVWriteArgs& a, int64_t i0, int64_t step) {
  const int per_row = VEC ? a.D / 8 : a.D;
  const int64_t total = (int64_t)a.num_seqs * a.hkv * per_row;
  for (int64_t i = i0; i < total; i += step) {
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

// Argument bundle of the prefill block copy: source rows [num_tokens, Hkv, D]
// with any element strides, written block by block into the caches.
struct PrefillCopyArgs {
  const uint16_t* key;
  int64_t ks_t, ks_h, ks_d;
  const uint16_t* val;
  int64_t vs_t, vs_h, vs_d;
  uint16_t* kc;
  int64_t kc_sb, kc_st, kc_sh;
  uint16_t* vc;
  int64_t vc_sb, vc_st, vc_sh;
  const int32_t* ids;  // destination block of each source block
  int num_ids, num_tokens, hkv, D, bs, num_blocks;
};

// Argument bundle of the fused rotary embedding + K/V write: q, key and value
// rows [num_seqs, heads, D] with any element strides, per-sequence cos/sin
// rows [num_seqs, D]; rotated queries go to q_out, rotated keys and values to
// the new token's cache slot.
struct RopeKVArgs {
  const uint16_t* q;
  int64_t qs_b, qs_h, qs_d;
  const uint16_t* key;
  int64_t ks_b, ks_h, ks_d;
  const uint16_t* val;
  int64_t vs_b, vs_h, vs_d;
  const uint16_t* cos;
  int64_t cs_b, cs_d;
  const uint16_t* sin;
  int64_t ss_b, ss_d;
  uint16_t* q_out;
  int64_t qo_b, qo_h;
  uint16_t* kc;
  int64_t kc_sb, kc_st, kc_sh;
  uint16_t* vc;
  int64_t vc_sb, vc_st, vc_sh;
  const int32_t* bt;
  int64_t bt_sb, bt_sk;
  const int32_t* lens;  // per-sequence lengths, or null: use uniform_len
  int uniform_len;
  int num_seqs, hq, hkv, D, bs, num_blocks, max_blocks;
};

// Argument bundle of the paged prefill attention: new query rows of all
// sequences packed [num_tokens, Hq, D] (sequence b owns rows qstart[b] ..
// qstart[b + 1]), each attending causally over its first lens[b] pool rows.
struct PrefillAttnArgs {
  const f16* q;
  int64_t q_st, q_sh;
  const f16* k;
  int64_t k_sb, k_st, k_sh;
  const f16* v;
  int64_t v_sb, v_st, v_sh;
  const int32_t* bt;
  int64_t bt_sb, bt_sk;
  const int32_t* lens;    // context length after the new tokens
  const int32_t* qstart;  // [num_seqs + 1] first query row of each sequence
  f16* out;
  int64_t o_st, o_sh;
  int num_seqs, num_tokens, hkv, g, bs, num_blocks, max_blocks;
  int col_blocks;  // column blocks per (sequence, kv head): ceil(max_query_len * g / columns)
  int col_groups;   // columns per workgroup in units of 64: 1 or 2
  int wave_groups;  // column groups of 16 per wavefront: 1, or 2 (half the wavefronts)
  float scale_log2;
  // Key-range split: a column block whose keys span more than split_tiles key
  // tiles is processed by several workgroups (up to max_splits), which leave
  // partial records; the last to finish merges them.
  int split_tiles, max_splits;
  int* cnt;     // per-column-block arrival counters, zero between launches
  float* recs;  // [seq][kv head][column block][split] records of (D + 2) x columns floats
};

// Columns of a prefill workgroup in units of 64 (token, query head) columns:
// two (128 columns) below head_dim 256, where the registers allow it. At head_dim
// 128 the kernel runs them as four wavefronts of two groups of 16 (each K and V
// operand read from LDS then feeds two MFMAs); up to head_dim 64 as either that
// or eight wavefronts of one group, chosen per launch by prefill_plan. Launches
// with few column blocks take one unit instead (twice the workgroups).
__host__ __device__ constexpr int prefill_col_groups(int D) { return D <= 128 ? 2 : 1; }
// The prefill workspace starts with a fixed region of arrival counters, one per
// column block of a split launch, so that the counters of every launch sit at
// the same place whatever its size and never overlap an earlier launch's
// records (launches that split have fewer column blocks than this).
constexpr int kPfMaxCounters = 16384;
constexpr size_t kPfCounterBytes = (size_t)kPfMaxCounters * sizeof(int);
// Keys per staged prefill tile: 128 up to head_dim 64, 64 above (two K and V
// buffers of 128 keys would leave no LDS for a second workgroup).
__host__ __device__ constexpr int prefill_key_tile(int D) { return D <= 64 ? 128 : 64; }

// Supplies the device address of a caller-less scratch buffer for the launch
// on `stream` (the no-allocation entry point's static array); returns a PA_*
// status.
typedef int (*ScratchFn)(void** ptr, hipStream_t stream);

// Batched decode attention behind pa_decode_batched_f16 (pa_capi.hip). With
// `scratch` set, the workspace is not the caller's: workspace_bytes is the
// size of the buffer `scratch` supplies, and calls that need more than that,
// or the fixed-split path, are refused.
struct RopeIn;
// With `newrow` set, the call first writes each sequence's new token (its key
// and value rows, newrow->key / newrow->val, at position seq_lens[b] - 1) into
// the pool -- in the attention launch itself where the planned kernel supports
// it, else as a K/V write launch before it.
int decode_batched(const void* q, const int64_t q_strides[3], const void* k_cache,
                   const int64_t k_strides[4], const void* v_cache, const int64_t v_strides[4],
                   const int32_t* block_tables, const int64_t bt_strides[2],
                   const int32_t* seq_lens, void* out, const int64_t out_strides[3],
                   int num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
                   int block_size, int num_blocks, int max_blocks_per_seq, float scale,
                   void* workspace, size_t workspace_bytes, ScratchFn scratch, void* stream,
                   const RopeIn* newrow = nullptr);

// Launchers (defined next to their kernels).
hipError_t launch_decode_split(const DecodeArgs& a, int D, int num_seqs, hipStream_t s);
hipError_t launch_decode_v1(const DecodeArgs& a, int D, hipStream_t s);
hipError_t launch_kv_write(const KVWriteArgs& a, bool vec, hipStream_t s);
hipError_t launch_prefill_copy(const PrefillCopyArgs& a, bool vec, hipStream_t s);
hipError_t launch_rope_kv_write(const RopeKVArgs& a, bool vec, hipStream_t s);
hipError_t launch_decode_streamk(const DecodeArgs& a, int D, hipStream_t s);
// Whether the stream-K kernel launched for `a` builds prefix items (block size
// 16 or 32, head_dim <= 64, pool strides its tile addressing covers, table
// strides for which 32 rows and 64 columns span less than 2^31 entries).
bool streamk_can_share(const DecodeArgs& a, int D);

// The new token's rows of a fused decode-layer call (decode_pair_kernel with
// rotary embedding): keys and values [num_seqs, kv heads, D] and the rotary
// cos / sin rows [num_seqs, D], all with unit head_dim stride, 16-byte aligned
// rows. Element strides.
struct RopeIn {
  const f16* key;
  int64_t ks_b, ks_h;
  const f16* val;
  int64_t vs_b, vs_h;
  const f16* cos;
  int64_t cs_b;
  const f16* sin;
  int64_t ss_b;
};
// Whether the fused decode-layer kernel serves the launch planned in `a`
// (one workgroup per pair, head_dim 64 or 128, block 16 or 32), and its
// launcher.
bool pair_rope_supported(const DecodeArgs& a, int D);
hipError_t launch_decode_pair_rope(const DecodeArgs& a, const RopeIn& r, int D, hipStream_t s);
// Whether the attention kernel with the K/V write in the same launch serves
// the launch planned in `a` (one workgroup per pair, head_dim 64 or 128,
// block 16 or 32; key and value rows in r.key / r.val, 16-byte aligned), and
// its launcher. Stream-K launches take the K/V write as a launch of its own:
// measured on MI355X at batch 256 x lognormal ~4.6k tokens, the write state
// inside decode_streamk_kernel (new rows substituted while staging, the slot
// written after the merge) cost 112.9 us per step against 100.9 us for the two
// launches (register spills in the segment walk).
bool decode_write_supported(const DecodeArgs& a, int D);
hipError_t launch_decode_write(const DecodeArgs& a, const RopeIn& r, int D, hipStream_t s);
// The K/V write of `w` in one launch with the stream-K plan of the planned
// launch `a` (written to a.plan_out), for an attention launch that follows it
// on the same stream with a.plan_in set (launch_decode_streamk then runs the
// kernel that reads the plan). Supported for stream-K ranges at head_dim 64 or
// 128 and block size 16 or 32.
bool plan_handover_supported(const DecodeArgs& a, int D);
hipError_t launch_kv_write_plan(const DecodeArgs& a, const KVWriteArgs& w, bool vec,
                                hipStream_t s);
hipError_t launch_prefill_attn(const PrefillAttnArgs& a, int D, hipStream_t s);
hipError_t launch_rmsnorm(const f16* x, int64_t xs, const f16* res, int64_t rs, f16* sum,
                          int64_t ss, const f16* w, f16* y, int64_t ys, int rows, int H,
                          float eps, hipStream_t s);
hipError_t launch_silu_mul(const f16* gu, int64_t gs, f16* out, int64_t os, int rows, int I,
                           bool vec, hipStream_t s);
hipError_t launch_top2(const f16* logits, int64_t ls, int rows, int V, int64_t* idx, float* top,
                       bool vec, hipStream_t s);

// Length of sequence b clamped to [0, max_blocks * bs].
__device__ inline int clamped_len(const DecodeArgs& a, int b) {
  int L = a.lens ? a.lens[b] : a.uniform_len;
  const int cap = a.max_blocks * a.bs;
  return L < 0 ? 0 : (L > cap ? cap : L);
}

__device__ inline int num_splits_for(int ntiles, int split_tiles) {
  return ntiles ? (ntiles + split_tiles - 1) / split_tiles : 1;
}

// Floats in one split-K partial record for head_dim D: 16 maxima (exp2 domain),
// 16 denominators, then 16 x D unnormalised accumulators (row = q head in group).
__host__ __device__ constexpr int record_floats(int D) { return 32 + 16 * D; }

}  // namespace pa
