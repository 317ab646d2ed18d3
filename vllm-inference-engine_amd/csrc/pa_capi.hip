// C ABI of the paged-attention library: argument checks, launch geometry and
// error reporting. Declarations: include/paged_attention.h.
#include <stdarg.h>
#include <atomic>
#include <stdio.h>

#include <string>

#include "../../include/paged_attention.h"
#include "pa_common.h"

namespace pa {

static thread_local std::string g_error;

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
}

void clear_error() { g_error.clear(); }

// Tiles (16 tokens) per split-K partition of the fixed-split path (batches larger
// than the stream-K plan holds).
constexpr int kSplitTilesBatched = 32;

static bool supported_head_dim(int D) { return D == 32 || D == 64 || D == 128 || D == 256; }

static int split_tiles_for(int base, int bs) {
  // Keep the block ids a split can touch within the LDS staging array.
  const int64_t cap = ((int64_t)(kMaxIds - 2) * bs) / 16;
  int64_t t = base < cap ? base : cap;
  return t < 1 ? 1 : (int)t;
}

static int64_t max_tiles_for(int max_blocks, int bs) {
  return ((int64_t)max_blocks * bs + 15) / 16;
}

static int64_t splits_for(int64_t tiles, int split_tiles) {
  return tiles <= 0 ? 1 : (tiles + split_tiles - 1) / split_tiles;
}

static bool aligned(const void* p, size_t n) { return ((uintptr_t)p % n) == 0; }

// Checks shared by every decode entry point. Mirrors the reference asserts
// (engine/kernels/paged_attention.py:266-281, :648-662) plus what the kernels
// need for 16-byte loads.
static int check_common(const void* q, const void* k, const void* v, const void* out,
                        const int64_t* k_strides, const int64_t* v_strides, int num_q_heads,
                        int num_kv_heads, int head_dim, int block_size, int num_blocks) {
  if (!q || !k || !v || !out || !k_strides || !v_strides) {
    set_error("null pointer argument");
    return PA_ERR_ARG;
  }
  if (num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads != 0) {
    set_error("num_q_heads (%d) must be divisible by num_kv_heads (%d)", num_q_heads, num_kv_heads);
    return PA_ERR_ARG;
  }
  if (num_q_heads / num_kv_heads > 16) {
    set_error("query group size %d > 16 is not built", num_q_heads / num_kv_heads);
    return PA_ERR_UNSUPPORTED;
  }
  if (!supported_head_dim(head_dim)) {
    set_error("head_dim %d not built (32, 64, 128, 256)", head_dim);
    return PA_ERR_UNSUPPORTED;
  }
  if (block_size <= 0 || num_blocks <= 0) {
    set_error("block_size (%d) and num_blocks (%d) must be positive", block_size, num_blocks);
    return PA_ERR_ARG;
  }
  for (int i = 0; i < 3; ++i) {
    if (k_strides[i] % 8 || v_strides[i] % 8 || k_strides[i] < 0 || v_strides[i] < 0) {
      set_error("cache strides must be non-negative multiples of 8 elements");
      return PA_ERR_ARG;
    }
  }
  if (k_strides[3] != 1 || v_strides[3] != 1) {
    set_error("cache head_dim stride must be 1");
    return PA_ERR_ARG;
  }
  if (!aligned(k, 16) || !aligned(v, 16) || !aligned(q, 16) || !aligned(out, 8)) {
    set_error("q/k_cache/v_cache must be 16-byte aligned and out 8-byte aligned");
    return PA_ERR_ARG;
  }
  return PA_OK;
}

static int finish_launch(hipError_t e) {
  if (e != hipSuccess) {
    set_error("HIP launch failed: %s", hipGetErrorString(e));
    return PA_ERR_HIP;
  }
  return PA_OK;
}

// Checks and fills the K/V write's arguments (the new rows [num_seqs, kv
// heads, D] of key and value go to each sequence's slot of position L - 1);
// `vec` tells whether every stride and base allows 16-byte copies. Returns a
// PA_* status with the message set.
static int kv_write_args(KVWriteArgs& a, bool& vec, const void* key, const int64_t key_strides[3],
                         const void* value, const int64_t value_strides[3], void* k_cache,
                         const int64_t k_strides[4], void* v_cache, const int64_t v_strides[4],
                         const int32_t* block_tables, const int64_t bt_strides[2],
                         const int32_t* seq_lens, int uniform_seq_len, int num_seqs,
                         int num_kv_heads, int head_dim, int block_size, int num_blocks,
                         int max_blocks_per_seq) {
  if (!key || !value || !k_cache || !v_cache || !key_strides || !value_strides || !k_strides ||
      !v_strides || !block_tables || !bt_strides) {
    set_error("null pointer argument");
    return PA_ERR_ARG;
  }
  if (num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 || num_blocks <= 0 ||
      max_blocks_per_seq <= 0) {
    set_error("num_kv_heads, head_dim, block_size, num_blocks and the table width must be "
              "positive");
    return PA_ERR_ARG;
  }
  if (k_strides[3] != 1 || v_strides[3] != 1) {
    set_error("cache head_dim stride must be 1");
    return PA_ERR_ARG;
  }
  a = KVWriteArgs{};
  a.key = (const uint16_t*)key;
  a.ks_b = key_strides[0];
  a.ks_h = key_strides[1];
  a.ks_d = key_strides[2];
  a.val = (const uint16_t*)value;
  a.vs_b = value_strides[0];
  a.vs_h = value_strides[1];
  a.vs_d = value_strides[2];
  a.kc = (uint16_t*)k_cache;
  a.kc_sb = k_strides[0];
  a.kc_st = k_strides[1];
  a.kc_sh = k_strides[2];
  a.vc = (uint16_t*)v_cache;
  a.vc_sb = v_strides[0];
  a.vc_st = v_strides[1];
  a.vc_sh = v_strides[2];
  a.bt = block_tables;
  a.bt_sb = bt_strides[0];
  a.bt_sk = bt_strides[1];
  a.lens = seq_lens;
  a.uniform_len = uniform_seq_len;
  a.num_seqs = num_seqs;
  a.hkv = num_kv_heads;
  a.D = head_dim;
  a.bs = block_size;
  a.num_blocks = num_blocks;
  a.max_blocks = max_blocks_per_seq;
  vec = head_dim % 8 == 0 && a.ks_d == 1 && a.vs_d == 1 && a.ks_b % 8 == 0 && a.ks_h % 8 == 0 &&
        a.vs_b % 8 == 0 && a.vs_h % 8 == 0 && a.kc_sb % 8 == 0 && a.kc_st % 8 == 0 &&
        a.kc_sh % 8 == 0 && a.vc_sb % 8 == 0 && a.vc_st % 8 == 0 && a.vc_sh % 8 == 0 &&
        aligned(key, 16) && aligned(value, 16) && aligned(k_cache, 16) && aligned(v_cache, 16);
  return PA_OK;
}

// ---- stream-K schedule: grid size and workspace layout ----

static int device_cus();

// Kv heads per stream-K pair. Two (head_dim <= 64, even kv-head count) fill 14
// of 16 MFMA columns at group size 7 and halve the tiles and pair segments,
// which pays when the batch's (sequence, kv head) pairs outnumber the CUs.
// Fewer pairs take one kv head each: twice the workgroups, each with half the
// work, shortens calls that are bound by their chain of memory round trips.
// Measured on MI355X (14 q / 2 kv heads, head_dim 64): batch 128 x 64 +
// U[64, 1024] tokens 25.1 -> 18.4 us per call; batch 1-32 x 128-2048 tokens
// 1-4 us faster; batch 256 x lognormal ~4.6k tokens 104 us with two, 112 with one.
static int streamk_head_group(int num_kv_heads, int D, int num_seqs) {
  return (D <= 64 && num_kv_heads % 2 == 0 && (int64_t)num_seqs * num_kv_heads > device_cus())
             ? 2 : 1;
}

// Upper bound of the workgroups a stream-K launch uses for these sizes (the
// grid never exceeds the number of tiles).
static int streamk_grid_bound(int num_seqs, int num_kv_heads, int head_dim, int block_size,
                              int max_blocks) {
  const int hg = streamk_head_group(num_kv_heads, head_dim, num_seqs);
  const int64_t tiles = (int64_t)(num_kv_heads / hg) * num_seqs * max_tiles_for(max_blocks, block_size);
  return (int)(tiles < kSkMaxWG ? (tiles < 1 ? 1 : tiles) : kSkMaxWG);
}

// Fewest sequences for which a launch looks for shared prefixes: finding the
// groups costs every workgroup about 2-3 us at the start of the launch
// (measured on MI355X), which only large batches recover.
constexpr int kShareMinSeqs = 64;

// Whether a launch over these sizes may build prefix items: head_dim <= 64,
// block size 16 or 32, at least kShareMinSeqs sequences (and, at launch, pool
// strides that the block-size-specialised kernels address and table strides
// the plan's 32-bit row offsets cover; see streamk_can_share).
static bool streamk_may_share(int num_seqs, int head_dim, int block_size) {
  return num_seqs >= kShareMinSeqs && head_dim <= 64 && (block_size == 16 || block_size == 32);
}

// Partial records of a launch of `grid` workgroups: two slots per workgroup of
// slot_recs records each, plus, with prefix items, one suffix and one prefix
// record per (sequence, kv head).
static size_t streamk_records_bytes(int num_seqs, int num_kv_heads, int head_dim, int grid,
                                    int slot_recs, bool share) {
  const size_t rec = (size_t)record_floats(head_dim) * sizeof(float);
  return (size_t)grid * 2 * slot_recs * rec +
         (share ? (size_t)2 * num_seqs * num_kv_heads * rec : 0);
}

// Stream-K workspace: the pair counters (kSkCounterBytes, zero between
// launches) followed by the partial records of the largest grid a launch over
// these sizes uses on the current device, with room for prefix items whenever
// the sizes allow them.
static size_t streamk_workspace(int num_seqs, int num_kv_heads, int head_dim, int block_size,
                                int max_blocks) {
  const int bound = streamk_grid_bound(num_seqs, num_kv_heads, head_dim, block_size, max_blocks);
  const int want = kSkWgPerCu * device_cus();
  const int grid = want < bound ? want : bound;  // the largest grid streamk_plan chooses
  const int hg = streamk_head_group(num_kv_heads, head_dim, num_seqs);
  const bool share = streamk_may_share(num_seqs, head_dim, block_size);
  const int slot_recs = share && kPfxColBlocks > hg ? kPfxColBlocks : hg;
  return kSkCounterBytes +
         streamk_records_bytes(num_seqs, num_kv_heads, head_dim, grid, slot_recs, share);
}

// The stream-K plan holds up to kSkMaxSeqs sequences in LDS and counts
// arrivals for up to kSkMaxPairs (sequence, kv-head group) pairs.
static bool streamk_ok(int num_seqs, int num_kv_heads, int head_dim) {
  const int hg = streamk_head_group(num_kv_heads, head_dim, num_seqs);
  return num_seqs <= kSkMaxSeqs && (int64_t)(num_kv_heads / hg) * num_seqs <= kSkMaxPairs;
}

// Longest pair (in 16-token tiles) that the one-workgroup-per-pair schedule takes.
constexpr int kPairTilesMax = 128;
// Tables of at most this many tiles keep one workgroup per pair, and a
// stream-K range takes at least kSkMinRange tile positions (tiles plus segment
// overhead). Measured on MI355X with the current kernels (14 q / 2 kv heads,
// head_dim 64, block 16, equal lengths, four pool copies rotated, rocprofv3
// kernel durations), one workgroup per pair against stream-K ranges: batch
// 1-32 x 512 tokens 6.5-8.1 us against 10.9-14.0 us; x 1024 tokens 8.3-11.3
// us against 11.8-15.1 us; x 2048 tokens 14.9-17.2 us against 12.8-17.5 us
// (batch 1-16 faster split). An earlier build with caches evicted: batch 1-32
// x 2048 33-35 us one per pair, 18-21 us split with ranges of at least 8
// positions (16: 19-21 us, 64: 25-30 us).
constexpr int kPairShortTiles = 64;
// Ranges of at least 16 positions against 8, 32 and 64 (same shapes, HIP events
// behind a GPU busy-wait, medians of 60 calls, one box): batch 1 x 2048 tokens
// 14.8 against 15.4, 15.0 and 17.1 us; 4 x 2048 15.1 against 16.3, 15.2 and
// 17.7; 1 x 4096 16.0 against 17.8, 16.2 and 17.1; 1 x 8192 18.7 against 23.2,
// 17.8 and 18.9; batches that fill the GPU unchanged.
constexpr int kSkMinRange = 16;

// Compute units of the current device (cached per device; threads that race
// on the first query store the same value).
static int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Fills the stream-K schedule fields of `a` (head group, grid, ranges) for a
// launch over num_seqs sequences; the workspace pointers are set at launch.
static void streamk_plan(DecodeArgs& a, int num_seqs, int head_dim) {
  const int bound = streamk_grid_bound(num_seqs, a.hkv, head_dim, a.bs, a.max_blocks);
  const int want = kSkWgPerCu * device_cus();
  a.num_seqs = num_seqs;
  a.num_wg = want < bound ? want : bound;
  // Pairs no longer than kPairTilesMax tiles (bounded by the table width) run
  // one per workgroup when they fill at least half the GPU, or when the table
  // holds at most kPairShortTiles tiles: splitting them would cost more in
  // segment starts and merges than it balances. Fewer, longer pairs are split
  // into ranges of at least kSkMinRange tile positions.
  a.head_group = streamk_head_group(a.hkv, head_dim, num_seqs);
  const int pairs = num_seqs * (a.hkv / a.head_group);
  const int64_t tmax = max_tiles_for(a.max_blocks, a.bs);
  a.pair_per_wg = pairs <= want && tmax <= kPairTilesMax &&
                  (2 * pairs >= want || tmax <= kPairShortTiles);
  if (a.pair_per_wg) a.num_wg = pairs;
  // A pair segment costs a workgroup about as long as streaming 176 KB of K/V
  // (pipeline fill, the drain and merge across wavefronts). Measured on MI355X
  // (HIP events behind a GPU busy-wait, A/B on one box), budgets of 240, 208,
  // 176 and 144 KB: long-context batch of 256 (lognormal ~4.6k tokens, shared
  // prefixes) 101.1-101.6, 99.3-99.5, 99.0-99.1, 100.2-100.4 us; batch 64 x
  // 2048 tokens at 7 kv heads, head_dim 128: 86.2, 85.3, 84.3-84.5, 84.2-84.3
  // us; other shapes within 0.3 us.
  const int tile_bytes = 64 * a.head_group * head_dim;
  a.seg_cost = (176 << 10) / tile_bytes;
  a.min_range = kSkMinRange;
  // Prefix items: only where ranges are used (one workgroup per pair cuts
  // nothing and merges nothing) and the kernel builds them.
  a.max_members = pfx_members(a.g);
  a.share = !a.pair_per_wg && streamk_may_share(num_seqs, head_dim, a.bs) &&
            streamk_can_share(a, head_dim);
  a.slot_recs = a.share && kPfxColBlocks > a.head_group ? kPfxColBlocks : a.head_group;
}

// Workspace bytes the planned launch touches: the pair counters, then two
// partial records per workgroup of its grid (at most what
// streamk_workspace() reserves for the same sizes).
static size_t streamk_need(const DecodeArgs& a, int head_dim) {
  return kSkCounterBytes + streamk_records_bytes(a.num_seqs, a.hkv, head_dim, a.num_wg,
                                                 a.slot_recs, a.share != 0);
}

// Launches a planned stream-K call; `ws` holds the pair counters then the
// records, ws_bytes of them (at least streamk_need()).
static hipError_t launch_streamk_planned(DecodeArgs& a, int head_dim, void* ws, size_t ws_bytes,
                                         hipStream_t s) {
  a.cnt = (int*)ws;
  a.recs = (float*)((char*)ws + kSkCounterBytes);
  const size_t rb = ws_bytes - kSkCounterBytes;
  a.recs_bytes = rb < 0x7fffffffu ? (int)rb : 0x7fffffff;
  return launch_decode_streamk(a, head_dim, s);
}

// ---- prefill attention: key-range split plan and workspace layout ----

// Fewest key tiles a split of the prefill kernel takes.
constexpr int kPrefillMinSplitTiles = 4;

struct PrefillPlan {
  int64_t col_blocks = 0, split_tiles = 1, max_splits = 1;
  int col_groups = 1, wave_groups = 1;
  size_t counter_bytes = 0, ws_bytes = 0;
};

// Fewer workgroups than this before any key-range split (with two column
// groups per wavefront): one column group instead, twice the workgroups.
// Measured on MI355X at head_dim 64, g = 7: one sequence of 2048 cached + 512
// new tokens (56 workgroups with two groups) 49.9 -> 33.4 us; at 112 and
// more workgroups two groups stay faster (8192 + 1024: 85.1 vs 92.4 us).
constexpr int64_t kPrefillFewBlocks = 64;

// Column blocks of `cols` (token, head) columns per (sequence, kv head). When
// they fill less than three quarters of the GPU's resident workgroup slots,
// each column block's key range is split into pieces of split_tiles key tiles
// (at least kPrefillMinSplitTiles) so that about that many workgroups exist. The
// workspace then holds the fixed counter region (kPfCounterBytes, one counter
// per column block, zero between launches) and a record of (head_dim + 2) x
// cols floats per split.
static PrefillPlan prefill_plan(int num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
                                int block_size, int max_blocks, int max_query_len) {
  PrefillPlan p;
  const int g = num_q_heads / num_kv_heads;
  p.col_groups = prefill_col_groups(head_dim);
  auto blocks_for = [&](int cg) { return ((int64_t)max_query_len * g + 64 * cg - 1) / (64 * cg); };
  if (p.col_groups > 1 && blocks_for(p.col_groups) * num_seqs * num_kv_heads < kPrefillFewBlocks)
    p.col_groups = 1;
  const int cols = 64 * p.col_groups;
  p.col_blocks = blocks_for(p.col_groups);
  const int kt = prefill_key_tile(head_dim);
  const int64_t max_tiles = ((int64_t)max_blocks * block_size + kt - 1) / kt;
  const int64_t base = p.col_blocks * num_seqs * num_kv_heads;
  // The kernel keeps two workgroups per CU resident (one at head_dim 256, for
  // LDS); splitting pays only while the column blocks fill less than about
  // three quarters of those slots.
  const int64_t target = (int64_t)device_cus() * (head_dim <= 128 ? 2 : 1) * 3 / 4;
  p.split_tiles = max_tiles < 1 ? 1 : max_tiles;
  if (base > 0 && base < target && base <= kPfMaxCounters && max_tiles > kPrefillMinSplitTiles) {
    const int64_t want = (target + base - 1) / base;
    int64_t st = (max_tiles + want - 1) / want;
    if (st < kPrefillMinSplitTiles) st = kPrefillMinSplitTiles;
    p.split_tiles = st;
    p.max_splits = (max_tiles + st - 1) / st;
  }
  // Up to head_dim 64, 128 columns run as four wavefronts of two column groups
  // (each LDS operand read feeds two MFMAs; two wavefronts per SIMD) or eight of
  // one group (four per SIMD). With workgroups of even length the first is
  // faster; where some finish early (the causal part is most of the context, or
  // the last piece of a split key range is short) a workgroup left alone on a CU
  // has one wavefront per SIMD in that form and the second is faster. At head_dim
  // 64 split pieces of 48 tiles and more are long enough for the first. Measured
  // on MI355X at g = 7, block 16 (back-to-back means of 30 calls, three
  // alternating rounds on one box): head_dim 64, 8 x (2048 + 512) 52.6-53.4 vs
  // 55.8-56.2 us, 4 x (8192 + 1024) 177.0-177.8 vs 187.3-188.7, 8 x (2048 +
  // 1024) 109.4-110.2 vs 114.4-114.8; 2 x 2048-token prompts 35.3-35.4 vs
  // 34.1-34.2, 8192 + 1024 split four ways (pieces of 18 tiles) 66.6-67.3 vs
  // 62.7-63.5; split two ways: 16384 + 2048 190.4-193.8 vs 199.2-201.3, 32768 +
  // 2048 344.9-346.6 vs 362.7-366.7, 12288 + 2048 151.7-152.4 vs 156.7-158.9;
  // 16384 + 1024 split four ways (34 tiles) 104.5-105.4 vs 104.8-105.2; head_dim
  // 32, 8 x (2048 + 512) 39.3-40.4 vs 40.0-42.2, 16384 + 2048 split two ways
  // 136.9-137.6 vs 134.7-135.6.
  constexpr int64_t kPrefillLongPieceTiles = 48;
  if (head_dim > 64)
    p.wave_groups = p.col_groups;
  else if (p.col_groups == 2 &&
           ((p.max_splits == 1 && 2 * (int64_t)max_query_len <= (int64_t)max_blocks * block_size) ||
            (p.max_splits > 1 && head_dim == 64 && p.split_tiles >= kPrefillLongPieceTiles)))
    p.wave_groups = 2;
  if (p.max_splits > 1) {
    p.counter_bytes = kPfCounterBytes;
    p.ws_bytes = p.counter_bytes +
                 (size_t)base * p.max_splits * cols * (head_dim + 2) * sizeof(float);
  }
  return p;
}

}  // namespace pa

using namespace pa;

extern "C" {

int pa_abi_version(void) { return 14; }

const char* pa_last_error(void) { return g_error.c_str(); }

size_t pa_decode_batched_workspace_bytes(int num_seqs, int num_q_heads, int num_kv_heads,
                                         int head_dim, int block_size, int max_blocks_per_seq) {
  (void)num_q_heads;
  if (num_seqs <= 0 || num_kv_heads <= 0 || block_size <= 0 || max_blocks_per_seq <= 0 ||
      !supported_head_dim(head_dim))
    return 0;
  if (streamk_ok(num_seqs, num_kv_heads, head_dim))
    return streamk_workspace(num_seqs, num_kv_heads, head_dim, block_size, max_blocks_per_seq);
  // The fixed-split records start after the counter region too, so that one
  // workspace can serve both paths without touching the stream-K counters.
  const int st = split_tiles_for(kSplitTilesBatched, block_size);
  const int64_t ms = splits_for(max_tiles_for(max_blocks_per_seq, block_size), st);
  if (ms <= 1) return 0;
  return kSkCounterBytes + (size_t)num_seqs * num_kv_heads * ms * record_floats(head_dim) * sizeof(float);
}

int pa_decode_batched_schedule(int num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
                               int block_size, int max_blocks_per_seq, int info[4]) {
  clear_error();
  if (!info || num_seqs <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 ||
      num_q_heads % num_kv_heads || num_q_heads / num_kv_heads > 16 || block_size <= 0 ||
      max_blocks_per_seq <= 0 || !supported_head_dim(head_dim)) {
    set_error("invalid or unsupported sizes");
    return PA_ERR_ARG;
  }
  if (!streamk_ok(num_seqs, num_kv_heads, head_dim)) {
    info[0] = 2;
    info[1] = 1;
    info[2] = num_seqs;
    info[3] = 0;
    return PA_OK;
  }
  DecodeArgs a{};
  a.hkv = num_kv_heads;
  a.g = num_q_heads / num_kv_heads;
  a.bs = block_size;
  a.max_blocks = max_blocks_per_seq;
  // A contiguous pool [num_blocks, block_size, num_kv_heads, head_dim].
  a.k_st = a.v_st = (int64_t)num_kv_heads * head_dim;
  a.k_sh = a.v_sh = head_dim;
  streamk_plan(a, num_seqs, head_dim);
  info[0] = a.pair_per_wg ? 1 : 0;
  info[1] = a.head_group;
  info[2] = a.num_wg;
  info[3] = a.share;
  return PA_OK;
}

int pa_decode_batched_f16(const void* q, const int64_t q_strides[3], const void* k_cache,
                          const int64_t k_strides[4], const void* v_cache,
                          const int64_t v_strides[4], const int32_t* block_tables,
                          const int64_t bt_strides[2], const int32_t* seq_lens, void* out,
                          const int64_t out_strides[3], int num_seqs, int num_q_heads,
                          int num_kv_heads, int head_dim, int block_size, int num_blocks,
                          int max_blocks_per_seq, float scale, void* workspace,
                          size_t workspace_bytes, void* stream) {
  clear_error();
  return pa::decode_batched(q, q_strides, k_cache, k_strides, v_cache, v_strides, block_tables,
                            bt_strides, seq_lens, out, out_strides, num_seqs, num_q_heads,
                            num_kv_heads, head_dim, block_size, num_blocks, max_blocks_per_seq,
                            scale, workspace, workspace_bytes, nullptr, stream);
}

int pa_decode_kv_write_batched_f16(const void* q, const int64_t q_strides[3], const void* key,
                                   const int64_t key_strides[3], const void* value,
                                   const int64_t value_strides[3], void* k_cache,
                                   const int64_t k_strides[4], void* v_cache,
                                   const int64_t v_strides[4], const int32_t* block_tables,
                                   const int64_t bt_strides[2], const int32_t* seq_lens,
                                   void* out, const int64_t out_strides[3], int num_seqs,
                                   int num_q_heads, int num_kv_heads, int head_dim,
                                   int block_size, int num_blocks, int max_blocks_per_seq,
                                   float scale, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  clear_error();
  if (num_seqs > 0 && (!key || !value || !key_strides || !value_strides)) {
    set_error("null pointer argument");
    return PA_ERR_ARG;
  }
  if (num_seqs > 0 && (key_strides[2] != 1 || value_strides[2] != 1 || key_strides[0] % 8 ||
                       key_strides[1] % 8 || value_strides[0] % 8 || value_strides[1] % 8 ||
                       !aligned(key, 16) || !aligned(value, 16))) {
    set_error("key/value rows need unit head_dim stride, 8-element aligned strides and 16-byte "
              "aligned bases");
    return PA_ERR_ARG;
  }
  RopeIn r{};
  r.key = (const f16*)key;
  r.ks_b = num_seqs > 0 ? key_strides[0] : 0;
  r.ks_h = num_seqs > 0 ? key_strides[1] : 0;
  r.val = (const f16*)value;
  r.vs_b = num_seqs > 0 ? value_strides[0] : 0;
  r.vs_h = num_seqs > 0 ? value_strides[1] : 0;
  return pa::decode_batched(q, q_strides, k_cache, k_strides, v_cache, v_strides, block_tables,
                            bt_strides, seq_lens, out, out_strides, num_seqs, num_q_heads,
                            num_kv_heads, head_dim, block_size, num_blocks, max_blocks_per_seq,
                            scale, workspace, workspace_bytes, nullptr, stream, &r);
}

}  // extern "C"

namespace pa {

int decode_batched(const void* q, const int64_t q_strides[3], const void* k_cache,
                   const int64_t k_strides[4], const void* v_cache, const int64_t v_strides[4],
                   const int32_t* block_tables, const int64_t bt_strides[2],
                   const int32_t* seq_lens, void* out, const int64_t out_strides[3],
                   int num_seqs, int num_q_heads, int num_kv_heads, int head_dim,
                   int block_size, int num_blocks, int max_blocks_per_seq, float scale,
                   void* workspace, size_t workspace_bytes, ScratchFn scratch, void* stream,
                   const RopeIn* newrow) {
  if (num_seqs < 0) {
    set_error("num_seqs must be >= 0");
    return PA_ERR_ARG;
  }
  if (num_seqs == 0) return PA_OK;
  int rc = check_common(q, k_cache, v_cache, out, k_strides, v_strides, num_q_heads,
                        num_kv_heads, head_dim, block_size, num_blocks);
  if (rc) return rc;
  if (!q_strides || !out_strides || !bt_strides || !block_tables || !seq_lens) {
    set_error("null pointer argument");
    return PA_ERR_ARG;
  }
  if (q_strides[2] != 1 || out_strides[2] != 1 || q_strides[0] % 8 || q_strides[1] % 8 ||
      out_strides[0] % 4 || out_strides[1] % 4) {
    set_error("q needs unit head_dim stride and 8-element aligned seq/head strides; "
              "out unit head_dim stride and 4-element aligned strides");
    return PA_ERR_ARG;
  }
  if (max_blocks_per_seq <= 0) {
    set_error("block table needs at least one column");
    return PA_ERR_ARG;
  }
  if (num_seqs > 65535) {
    set_error("num_seqs %d exceeds the grid limit 65535", num_seqs);
    return PA_ERR_UNSUPPORTED;
  }
  const int st = split_tiles_for(kSplitTilesBatched, block_size);
  const int64_t ms = splits_for(max_tiles_for(max_blocks_per_seq, block_size), st);
  const bool streamk = streamk_ok(num_seqs, num_kv_heads, head_dim);
  if (scratch && !streamk) {
    set_error("the no-allocation entry point takes at most %d sequences and %d (sequence, "
              "kv-head group) pairs; %d sequences of %d kv heads given",
              kSkMaxSeqs, kSkMaxPairs, num_seqs, num_kv_heads);
    return PA_ERR_UNSUPPORTED;
  }
  DecodeArgs a{};
  a.q = (const f16*)q;
  a.q_sb = q_strides[0];
  a.q_sh = q_strides[1];
  a.k = (const f16*)k_cache;
  a.k_sb = k_strides[0];
  a.k_st = k_strides[1];
  a.k_sh = k_strides[2];
  a.v = (const f16*)v_cache;
  a.v_sb = v_strides[0];
  a.v_st = v_strides[1];
  a.v_sh = v_strides[2];
  a.bt = block_tables;
  a.bt_sb = bt_strides[0];
  a.bt_sk = bt_strides[1];
  a.lens = seq_lens;
  a.uniform_len = 0;
  a.out = (f16*)out;
  a.o_sb = out_strides[0];
  a.o_sh = out_strides[1];
  a.ws = workspace ? (float*)((char*)workspace + kSkCounterBytes) : nullptr;
  a.hkv = num_kv_heads;
  a.g = num_q_heads / num_kv_heads;
  a.bs = block_size;
  a.num_blocks = num_blocks;
  a.max_blocks = max_blocks_per_seq;
  a.split_tiles = st;
  a.max_splits = (int)ms;
  a.scale_log2 = scale * kLog2e;
  // The new token's rows as a K/V write launch ahead of the attention launch.
  auto write_first = [&]() -> int {
    const int64_t ks[3] = {newrow->ks_b, newrow->ks_h, 1};
    const int64_t vs[3] = {newrow->vs_b, newrow->vs_h, 1};
    const int rc = pa_kv_write_f16(newrow->key, ks, newrow->val, vs, const_cast<void*>(k_cache),
                                   k_strides, const_cast<void*>(v_cache), v_strides, block_tables,
                                   bt_strides, seq_lens, 0, num_seqs, num_kv_heads, head_dim,
                                   block_size, num_blocks, max_blocks_per_seq, stream);
    return rc;
  };
  if (!streamk) {
    const size_t need = pa_decode_batched_workspace_bytes(num_seqs, num_q_heads, num_kv_heads,
                                                          head_dim, block_size, max_blocks_per_seq);
    if (need && (!workspace || workspace_bytes < need)) {
      set_error("workspace of %zu bytes needed, %zu given", need, workspace_bytes);
      return PA_ERR_WORKSPACE;
    }
    if (newrow) {
      const int rc = write_first();
      if (rc) return rc;
    }
    return finish_launch(launch_decode_split(a, head_dim, num_seqs, (hipStream_t)stream));
  }
  streamk_plan(a, num_seqs, head_dim);
  size_t need = streamk_need(a, head_dim);
  if (scratch && need > workspace_bytes && a.share) {
    // The fixed buffer cannot hold the prefix items' records: read shared
    // prefixes once per sequence instead.
    a.share = 0;
    a.slot_recs = a.head_group;
    need = streamk_need(a, head_dim);
  }
  if (scratch) {
    // The caller cannot allocate: the library's own fixed buffer, if it is large enough.
    if (need > workspace_bytes) {
      set_error("this call needs %zu bytes of scratch; the no-allocation entry point has %zu",
                need, workspace_bytes);
      return PA_ERR_UNSUPPORTED;
    }
    const int rc = scratch(&workspace, (hipStream_t)stream);
    if (rc) return rc;
  } else if (!workspace || workspace_bytes < need) {
    const size_t reserve = pa_decode_batched_workspace_bytes(
        num_seqs, num_q_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq);
    set_error("workspace of %zu bytes needed, %zu given", reserve, workspace_bytes);
    return PA_ERR_WORKSPACE;
  }
  if (newrow) {
    if (decode_write_supported(a, head_dim)) {
      a.cnt = (int*)workspace;
      a.recs = (float*)((char*)workspace + kSkCounterBytes);
      const size_t rb = workspace_bytes - kSkCounterBytes;
      a.recs_bytes = rb < 0x7fffffffu ? (int)rb : 0x7fffffff;
      return finish_launch(launch_decode_write(a, *newrow, head_dim, (hipStream_t)stream));
    }
    if (!plan_handover_supported(a, head_dim)) {
      const int rc = write_first();
      if (rc) return rc;
    } else {
      // Stream-K ranges: the K/V write launch also derives the plan once and
      // leaves it in the workspace head for the attention launch, instead of
      // every attention workgroup deriving it.
      const int64_t ks[3] = {newrow->ks_b, newrow->ks_h, 1};
      const int64_t vs[3] = {newrow->vs_b, newrow->vs_h, 1};
      KVWriteArgs w;
      bool vec = false;
      int rc = kv_write_args(w, vec, newrow->key, ks, newrow->val, vs, const_cast<void*>(k_cache),
                             k_strides, const_cast<void*>(v_cache), v_strides, block_tables,
                             bt_strides, seq_lens, 0, num_seqs, num_kv_heads, head_dim,
                             block_size, num_blocks, max_blocks_per_seq);
      if (rc) return rc;
      a.plan_out = (int*)((char*)workspace + kSkPairCounterBytes);
      rc = finish_launch(launch_kv_write_plan(a, w, vec, (hipStream_t)stream));
      if (rc) return rc;
      a.plan_in = a.plan_out;
      a.plan_out = nullptr;
    }
  }
  return finish_launch(launch_streamk_planned(a, head_dim, workspace, workspace_bytes,
                                              (hipStream_t)stream));
}

}  // namespace pa

extern "C" {

// Shared by the single-sequence entry points.
static int fill_single(DecodeArgs& a, const void* q, const int64_t q_strides[2],
                       const void* k_cache, const int64_t k_strides[4], const void* v_cache,
                       const int64_t v_strides[4], const int32_t* block_table, int64_t bt_stride,
                       int table_len, int seq_len, void* out, const int64_t out_strides[2],
                       int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                       int num_blocks, float scale) {
  int rc = check_common(q, k_cache, v_cache, out, k_strides, v_strides, num_q_heads,
                        num_kv_heads, head_dim, block_size, num_blocks);
  if (rc) return rc;
  if (!q_strides || !out_strides || !block_table) {
    set_error("null pointer argument");
    return PA_ERR_ARG;
  }
  if (q_strides[1] != 1 || out_strides[1] != 1 || q_strides[0] % 8 || out_strides[0] % 4) {
    set_error("q/out need unit head_dim stride and aligned head strides");
    return PA_ERR_ARG;
  }
  if (seq_len < 0) {
    set_error("seq_len must be >= 0");
    return PA_ERR_ARG;
  }
  const int64_t need_blocks = ((int64_t)seq_len + block_size - 1) / block_size;
  if (table_len < need_blocks || table_len <= 0) {
    set_error("block_table size (%d) smaller than needed (%lld)", table_len,
              (long long)need_blocks);
    return PA_ERR_ARG;
  }
  a = DecodeArgs{};
  a.q = (const f16*)q;
  a.q_sb = 0;
  a.q_sh = q_strides[0];
  a.k = (const f16*)k_cache;
  a.k_sb = k_strides[0];
  a.k_st = k_strides[1];
  a.k_sh = k_strides[2];
  a.v = (const f16*)v_cache;
  a.v_sb = v_strides[0];
  a.v_st = v_strides[1];
  a.v_sh = v_strides[2];
  a.bt = block_table;
  a.bt_sb = 0;
  a.bt_sk = bt_stride;
  a.lens = nullptr;
  a.uniform_len = seq_len;
  a.out = (f16*)out;
  a.o_sb = 0;
  a.o_sh = out_strides[0];
  a.hkv = num_kv_heads;
  a.g = num_q_heads / num_kv_heads;
  a.bs = block_size;
  a.num_blocks = num_blocks;
  a.max_blocks = table_len;
  a.scale_log2 = scale * kLog2e;
  return PA_OK;
}

size_t pa_decode_v2_workspace_bytes(int num_q_heads, int num_kv_heads, int head_dim,
                                    int block_size, int table_len) {
  (void)num_q_heads;
  if (num_kv_heads <= 0 || block_size <= 0 || table_len <= 0 || !supported_head_dim(head_dim))
    return 0;
  return streamk_workspace(1, num_kv_heads, head_dim, block_size, table_len);
}

int pa_decode_v2_f16(const void* q, const int64_t q_strides[2], const void* k_cache,
                     const int64_t k_strides[4], const void* v_cache, const int64_t v_strides[4],
                     const int32_t* block_table, int64_t bt_stride, int table_len, int seq_len,
                     void* out, const int64_t out_strides[2], int num_q_heads, int num_kv_heads,
                     int head_dim, int block_size, int num_blocks, float scale, void* workspace,
                     size_t workspace_bytes, void* stream) {
  clear_error();
  DecodeArgs a;
  int rc = fill_single(a, q, q_strides, k_cache, k_strides, v_cache, v_strides, block_table,
                       bt_stride, table_len, seq_len, out, out_strides, num_q_heads, num_kv_heads,
                       head_dim, block_size, num_blocks, scale);
  if (rc) return rc;
  streamk_plan(a, 1, head_dim);
  if (!workspace || workspace_bytes < streamk_need(a, head_dim)) {
    const size_t reserve =
        pa_decode_v2_workspace_bytes(num_q_heads, num_kv_heads, head_dim, block_size, table_len);
    set_error("workspace of %zu bytes needed, %zu given", reserve, workspace_bytes);
    return PA_ERR_WORKSPACE;
  }
  return finish_launch(launch_streamk_planned(a, head_dim, workspace, workspace_bytes,
                                              (hipStream_t)stream));
}

size_t pa_decode_v1_workspace_bytes(int num_q_heads, int num_kv_heads, int head_dim,
                                    int block_size, int seq_len) {
  (void)num_q_heads;
  (void)head_dim;
  (void)block_size;
  if (num_kv_heads <= 0 || seq_len <= 0) return 0;
  const int64_t lpad = ((int64_t)seq_len + 15) / 16 * 16;
  return (size_t)num_kv_heads * 16 * lpad * sizeof(float);
}

int pa_decode_v1_f16(const void* q, const int64_t q_strides[2], const void* k_cache,
                     const int64_t k_strides[4], const void* v_cache, const int64_t v_strides[4],
                     const int32_t* block_table, int64_t bt_stride, int table_len, int seq_len,
                     void* out, const int64_t out_strides[2], int num_q_heads, int num_kv_heads,
                     int head_dim, int block_size, int num_blocks, float scale, void* workspace,
                     size_t workspace_bytes, void* stream) {
  clear_error();
  DecodeArgs a;
  int rc = fill_single(a, q, q_strides, k_cache, k_strides, v_cache, v_strides, block_table,
                       bt_stride, table_len, seq_len, out, out_strides, num_q_heads, num_kv_heads,
                       head_dim, block_size, num_blocks, scale);
  if (rc) return rc;
  const size_t need =
      pa_decode_v1_workspace_bytes(num_q_heads, num_kv_heads, head_dim, block_size, seq_len);
  if (need && (!workspace || workspace_bytes < need)) {
    set_error("workspace of %zu bytes needed, %zu given", need, workspace_bytes);
    return PA_ERR_WORKSPACE;
  }
  a.ws = (float*)workspace;
  a.lpad = (int)(((int64_t)seq_len + 15) / 16 * 16);
  return finish_launch(launch_decode_v1(a, head_dim, (hipStream_t)stream));
}

int pa_kv_write_f16(const void* key, const int64_t key_strides[3], const void* value,
                    const int64_t value_strides[3], void* k_cache, const int64_t k_strides[4],
                    void* v_cache, const int64_t v_strides[4], const int32_t* block_tables,
                    const int64_t bt_strides[2], const int32_t* seq_lens, int uniform_seq_len,
                    int num_seqs, int num_kv_heads, int head_dim, int block_size, int num_blocks,
                    int max_blocks_per_seq, void* stream) {
  clear_error();
  if (num_seqs < 0) {
    set_error("num_seqs must be >= 0");
    return PA_ERR_ARG;
  }
  if (num_seqs == 0) return PA_OK;
  KVWriteArgs a;
  bool vec = false;
  const int rc = kv_write_args(a, vec, key, key_strides, value, value_strides, k_cache, k_strides,
                               v_cache, v_strides, block_tables, bt_strides, seq_lens,
                               uniform_seq_len, num_seqs, num_kv_heads, head_dim, block_size,
                               num_blocks, max_blocks_per_seq);
  if (rc) return rc;
  return finish_launch(launch_kv_write(a, vec, (hipStream_t)stream));
}

int pa_prefill_copy_f16(const void* key, const int64_t key_strides[3], const void* value,
                        const int64_t value_strides[3], void* k_cache, const int64_t k_strides[4],
                        void* v_cache, const int64_t v_strides[4], const int32_t* block_ids,
                        int num_block_ids, int num_tokens, int num_kv_heads, int head_dim,
                        int block_size, int num_blocks, void* stream) {
  clear_error();
  if (num_block_ids < 0 || num_tokens < 0) {
    set_error("num_block_ids and num_tokens must be >= 0");
    return PA_ERR_ARG;
  }
  if (num_block_ids == 0) return PA_OK;
  if ((int64_t)num_tokens > (int64_t)num_block_ids * block_size) {
    set_error("num_tokens (%d) exceeds the %d blocks given", num_tokens, num_block_ids);
    return PA_ERR_ARG;
  }
  if (!k_cache || !v_cache || !key_strides || !value_strides || !k_strides || !v_strides ||
      !block_ids || (num_tokens > 0 && (!key || !value))) {
    set_error("null pointer argument");
    return PA_ERR_ARG;
  }
  if (num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 || num_blocks <= 0) {
    set_error("num_kv_heads, head_dim, block_size and num_blocks must be positive");
    return PA_ERR_ARG;
  }
  if (k_strides[3] != 1 || v_strides[3] != 1) {
    set_error("cache head_dim stride must be 1");
    return PA_ERR_ARG;
  }
  PrefillCopyArgs a{};
  a.key = (const uint16_t*)key;
  a.ks_t = key_strides[0];
  a.ks_h = key_strides[1];
  a.ks_d = key_strides[2];
  a.val = (const uint16_t*)value;
  a.vs_t = value_strides[0];
  a.vs_h = value_strides[1];
  a.vs_d = value_strides[2];
  a.kc = (uint16_t*)k_cache;
  a.kc_sb = k_strides[0];
  a.kc_st = k_strides[1];
  a.kc_sh = k_strides[2];
  a.vc = (uint16_t*)v_cache;
  a.vc_sb = v_strides[0];
  a.vc_st = v_strides[1];
  a.vc_sh = v_strides[2];
  a.ids = block_ids;
  a.num_ids = num_block_ids;
  a.num_tokens = num_tokens;
  a.hkv = num_kv_heads;
  a.D = head_dim;
  a.bs = block_size;
  a.num_blocks = num_blocks;
  const bool vec = head_dim % 8 == 0 && a.ks_d == 1 && a.vs_d == 1 && a.ks_t % 8 == 0 &&
                   a.ks_h % 8 == 0 && a.vs_t % 8 == 0 && a.vs_h % 8 == 0 && a.kc_sb % 8 == 0 &&
                   a.kc_st % 8 == 0 && a.kc_sh % 8 == 0 && a.vc_sb % 8 == 0 &&
                   a.vc_st % 8 == 0 && a.vc_sh % 8 == 0 && aligned(key, 16) &&
                   aligned(value, 16) && aligned(k_cache, 16) && aligned(v_cache, 16);
  return finish_launch(launch_prefill_copy(a, vec, (hipStream_t)stream));
}


int pa_rope_kv_write_f16(const void* q, const int64_t q_strides[3], const void* key,
                         const int64_t key_strides[3], const void* value,
                         const int64_t value_strides[3], const void* cos,
                         const int64_t cos_strides[2], const void* sin,
                         const int64_t sin_strides[2], void* q_out,
                         const int64_t q_out_strides[3], void* k_cache,
                         const int64_t k_strides[4], void* v_cache, const int64_t v_strides[4],
                         const int32_t* block_tables, const int64_t bt_strides[2],
                         const int32_t* seq_lens, int uniform_seq_len, int num_seqs,
                         int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                         int num_blocks, int max_blocks_per_seq, void* stream) {
  clear_error();
  if (num_seqs < 0) {
    set_error("num_seqs must be >= 0");
    return PA_ERR_ARG;
  }
  if (num_seqs == 0) return PA_OK;
  if (!q || !key || !value || !cos || !sin || !q_out || !k_cache || !v_cache || !q_strides ||
      !key_strides || !value_strides || !cos_strides || !sin_strides || !q_out_strides ||
      !k_strides || !v_strides || !block_tables || !bt_strides) {
    set_error("null pointer argument");
    return PA_ERR_ARG;
  }
  if (num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || head_dim % 2 || block_size <= 0 ||
      num_blocks <= 0 || max_blocks_per_seq <= 0) {
    set_error("heads, an even head_dim, block_size, num_blocks and the table width must be "
              "positive");
    return PA_ERR_ARG;
  }
  if (k_strides[3] != 1 || v_strides[3] != 1 || q_out_strides[2] != 1) {
    set_error("cache and q_out head_dim stride must be 1");
    return PA_ERR_ARG;
  }
  RopeKVArgs a{};
  a.q = (const uint16_t*)q;
  a.qs_b = q_strides[0];
  a.qs_h = q_strides[1];
  a.qs_d = q_strides[2];
  a.key = (const uint16_t*)key;
  a.ks_b = key_strides[0];
  a.ks_h = key_strides[1];
  a.ks_d = key_strides[2];
  a.val = (const uint16_t*)value;
  a.vs_b = value_strides[0];
  a.vs_h = value_strides[1];
  a.vs_d = value_strides[2];
  a.cos = (const uint16_t*)cos;
  a.cs_b = cos_strides[0];
  a.cs_d = cos_strides[1];
  a.sin = (const uint16_t*)sin;
  a.ss_b = sin_strides[0];
  a.ss_d = sin_strides[1];
  a.q_out = (uint16_t*)q_out;
  a.qo_b = q_out_strides[0];
  a.qo_h = q_out_strides[1];
  a.kc = (uint16_t*)k_cache;
  a.kc_sb = k_strides[0];
  a.kc_st = k_strides[1];
  a.kc_sh = k_strides[2];
  a.vc = (uint16_t*)v_cache;
  a.vc_sb = v_strides[0];
  a.vc_st = v_strides[1];
  a.vc_sh = v_strides[2];
  a.bt = block_tables;
  a.bt_sb = bt_strides[0];
  a.bt_sk = bt_strides[1];
  a.lens = seq_lens;
  a.uniform_len = uniform_seq_len;
  a.num_seqs = num_seqs;
  a.hq = num_q_heads;
  a.hkv = num_kv_heads;
  a.D = head_dim;
  a.bs = block_size;
  a.num_blocks = num_blocks;
  a.max_blocks = max_blocks_per_seq;
  auto rows16 = [](const void* p, int64_t sb, int64_t sh, int64_t sd) {
    return aligned(p, 16) && sd == 1 && sb % 8 == 0 && sh % 8 == 0;
  };
  const bool vec = head_dim % 16 == 0 && rows16(q, a.qs_b, a.qs_h, a.qs_d) &&
                   rows16(key, a.ks_b, a.ks_h, a.ks_d) && rows16(value, a.vs_b, a.vs_h, a.vs_d) &&
                   rows16(cos, a.cs_b, 0, a.cs_d) && rows16(sin, a.ss_b, 0, a.ss_d) &&
                   rows16(q_out, a.qo_b, a.qo_h, 1) && rows16(k_cache, a.kc_sb, a.kc_st, 1) &&
                   a.kc_sh % 8 == 0 && rows16(v_cache, a.vc_sb, a.vc_st, 1) && a.vc_sh % 8 == 0;
  return finish_launch(launch_rope_kv_write(a, vec, (hipStream_t)stream));
}

size_t pa_decode_rope_batched_workspace_bytes(int num_seqs, int num_q_heads, int num_kv_heads,
                                              int head_dim, int block_size,
                                              int max_blocks_per_seq) {
  if (num_seqs <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || block_size <= 0 ||
      max_blocks_per_seq <= 0 || !supported_head_dim(head_dim))
    return 0;
  // The decode workspace, then room for the rotated queries of the two-launch
  // form (used when the one-launch kernel does not serve the shape).
  const size_t ws = pa_decode_batched_workspace_bytes(num_seqs, num_q_heads, num_kv_heads,
                                                      head_dim, block_size, max_blocks_per_seq);
  return ((ws + 255) & ~(size_t)255) + (size_t)num_seqs * num_q_heads * head_dim * 2;
}

int pa_decode_rope_batched_f16(const void* q, const int64_t q_strides[3], const void* key,
                               const int64_t key_strides[3], const void* value,
                               const int64_t value_strides[3], const void* cos,
                               const int64_t cos_strides[2], const void* sin,
                               const int64_t sin_strides[2], void* k_cache,
                               const int64_t k_strides[4], void* v_cache,
                               const int64_t v_strides[4], const int32_t* block_tables,
                               const int64_t bt_strides[2], const int32_t* seq_lens, void* out,
                               const int64_t out_strides[3], int num_seqs, int num_q_heads,
                               int num_kv_heads, int head_dim, int block_size, int num_blocks,
                               int max_blocks_per_seq, float scale, void* workspace,
                               size_t workspace_bytes, void* stream) {
  clear_error();
  if (num_seqs < 0) {
    set_error("num_seqs must be >= 0");
    return PA_ERR_ARG;
  }
  if (num_seqs == 0) return PA_OK;
  if (!q || !key || !value || !cos || !sin || !k_cache || !v_cache || !out || !q_strides ||
      !key_strides || !value_strides || !cos_strides || !sin_strides || !k_strides ||
      !v_strides || !block_tables || !bt_strides || !seq_lens || !out_strides) {
    set_error("null pointer argument");
    return PA_ERR_ARG;
  }
  int rc = check_common(q, k_cache, v_cache, out, k_strides, v_strides, num_q_heads, num_kv_heads,
                        head_dim, block_size, num_blocks);
  if (rc) return rc;
  // What pa_decode_batched_f16 requires of the table and the output holds for
  // both forms (q may have any strides: the two-launch form rotates it into a
  // contiguous copy, and the one-launch form is taken only for aligned rows).
  if (max_blocks_per_seq <= 0) {
    set_error("block table needs at least one column");
    return PA_ERR_ARG;
  }
  if (out_strides[2] != 1 || out_strides[0] % 4 || out_strides[1] % 4) {
    set_error("out needs unit head_dim stride and 4-element aligned strides");
    return PA_ERR_ARG;
  }
  if (num_seqs > 65535) {
    set_error("num_seqs %d exceeds the grid limit 65535", num_seqs);
    return PA_ERR_UNSUPPORTED;
  }
  const size_t ws_need = pa_decode_rope_batched_workspace_bytes(
      num_seqs, num_q_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq);
  if (!workspace || workspace_bytes < ws_need) {
    set_error("workspace of %zu bytes needed, %zu given", ws_need, workspace_bytes);
    return PA_ERR_WORKSPACE;
  }
  const size_t dec_ws = pa_decode_batched_workspace_bytes(num_seqs, num_q_heads, num_kv_heads,
                                                          head_dim, block_size, max_blocks_per_seq);
  // One launch when the batch takes one workgroup per (sequence, kv-head group)
  // and every row the kernel reads with 16-byte loads is so aligned.
  auto rows16 = [](const void* p, int64_t sb, int64_t sh, int64_t sd) {
    return aligned(p, 16) && sd == 1 && sb % 8 == 0 && sh % 8 == 0;
  };
  DecodeArgs a{};
  a.hkv = num_kv_heads;
  a.g = num_q_heads / num_kv_heads;
  a.bs = block_size;
  a.max_blocks = max_blocks_per_seq;
  a.k_st = k_strides[1];
  a.k_sh = k_strides[2];
  a.v_st = v_strides[1];
  a.v_sh = v_strides[2];
  streamk_plan(a, num_seqs, head_dim);
  const bool one_launch =
      num_seqs <= kSkMaxSeqs && pair_rope_supported(a, head_dim) &&
      rows16(q, q_strides[0], q_strides[1], q_strides[2]) &&
      rows16(key, key_strides[0], key_strides[1], key_strides[2]) &&
      rows16(value, value_strides[0], value_strides[1], value_strides[2]) &&
      rows16(cos, cos_strides[0], 0, cos_strides[1]) && rows16(sin, sin_strides[0], 0, sin_strides[1]) &&
      out_strides[2] == 1 && out_strides[0] % 4 == 0 && out_strides[1] % 4 == 0;
  if (!one_launch) {
    // Two launches: rotation and K/V write, then attention on the rotated queries.
    void* q_rot = (char*)workspace + ((dec_ws + 255) & ~(size_t)255);
    const int64_t qr_strides[3] = {(int64_t)num_q_heads * head_dim, head_dim, 1};
    rc = pa_rope_kv_write_f16(q, q_strides, key, key_strides, value, value_strides, cos, cos_strides,
                              sin, sin_strides, q_rot, qr_strides, k_cache, k_strides, v_cache,
                              v_strides, block_tables, bt_strides, seq_lens, 0, num_seqs,
                              num_q_heads, num_kv_heads, head_dim, block_size, num_blocks,
                              max_blocks_per_seq, stream);
    if (rc) return rc;
    return pa::decode_batched(q_rot, qr_strides, k_cache, k_strides, v_cache, v_strides,
                              block_tables, bt_strides, seq_lens, out, out_strides, num_seqs,
                              num_q_heads, num_kv_heads, head_dim, block_size, num_blocks,
                              max_blocks_per_seq, scale, workspace, dec_ws, nullptr, stream);
  }
  a.q = (const f16*)q;
  a.q_sb = q_strides[0];
  a.q_sh = q_strides[1];
  a.k = (const f16*)k_cache;
  a.k_sb = k_strides[0];
  a.v = (const f16*)v_cache;
  a.v_sb = v_strides[0];
  a.bt = block_tables;
  a.bt_sb = bt_strides[0];
  a.bt_sk = bt_strides[1];
  a.lens = seq_lens;
  a.out = (f16*)out;
  a.o_sb = out_strides[0];
  a.o_sh = out_strides[1];
  a.num_blocks = num_blocks;
  a.scale_log2 = scale * kLog2e;
  RopeIn r{};
  r.key = (const f16*)key;
  r.ks_b = key_strides[0];
  r.ks_h = key_strides[1];
  r.val = (const f16*)value;
  r.vs_b = value_strides[0];
  r.vs_h = value_strides[1];
  r.cos = (const f16*)cos;
  r.cs_b = cos_strides[0];
  r.sin = (const f16*)sin;
  r.ss_b = sin_strides[0];
  return finish_launch(launch_decode_pair_rope(a, r, head_dim, (hipStream_t)stream));
}

size_t pa_prefill_attention_workspace_bytes(int num_seqs, int num_q_heads, int num_kv_heads,
                                            int head_dim, int block_size,
                                            int max_blocks_per_seq, int max_query_len) {
  if (num_seqs <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads ||
      block_size <= 0 || max_blocks_per_seq <= 0 || max_query_len <= 0 ||
      !supported_head_dim(head_dim))
    return 0;
  return prefill_plan(num_seqs, num_q_heads, num_kv_heads, head_dim, block_size,
                      max_blocks_per_seq, max_query_len).ws_bytes;
}

int pa_prefill_attention_f16(const void* q, const int64_t q_strides[3], const void* k_cache,
                             const int64_t k_strides[4], const void* v_cache,
                             const int64_t v_strides[4], const int32_t* block_tables,
                             const int64_t bt_strides[2], const int32_t* seq_lens,
                             const int32_t* query_start_loc, int max_query_len, void* out,
                             const int64_t out_strides[3], int num_seqs, int num_tokens,
                             int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                             int num_blocks, int max_blocks_per_seq, float scale,
                             void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if (num_seqs < 0 || num_tokens < 0 || max_query_len < 0) {
    set_error("num_seqs, num_tokens and max_query_len must be >= 0");
    return PA_ERR_ARG;
  }
  if (num_seqs == 0 || num_tokens == 0 || max_query_len == 0) return PA_OK;
  int rc = check_common(q, k_cache, v_cache, out, k_strides, v_strides, num_q_heads,
                        num_kv_heads, head_dim, block_size, num_blocks);
  if (rc) return rc;
  if (!q_strides || !out_strides || !bt_strides || !block_tables || !seq_lens ||
      !query_start_loc) {
    set_error("null pointer argument");
    return PA_ERR_ARG;
  }
  if (q_strides[2] != 1 || out_strides[2] != 1 || q_strides[0] % 8 || q_strides[1] % 8 ||
      out_strides[0] % 4 || out_strides[1] % 4) {
    set_error("q needs unit head_dim stride and 8-element aligned token/head strides; "
              "out unit head_dim stride and 4-element aligned strides");
    return PA_ERR_ARG;
  }
  if (max_blocks_per_seq <= 0) {
    set_error("block table needs at least one column");
    return PA_ERR_ARG;
  }
  if (!(scale > 0.f) || scale == __builtin_huge_valf()) {
    set_error("scale must be positive and finite");
    return PA_ERR_ARG;
  }
  // The kernel's per-piece address arithmetic is 32-bit inside a block.
  const int64_t lim = 0x7fffffff;
  if (k_strides[0] > 0xffffffffll || v_strides[0] > 0xffffffffll ||
      k_strides[1] * block_size + head_dim > lim || v_strides[1] * block_size + head_dim > lim ||
      bt_strides[1] < 0 || bt_strides[1] * (int64_t)max_blocks_per_seq > lim) {
    set_error("cache block stride must fit 32 bits and row / table offsets 31 bits");
    return PA_ERR_UNSUPPORTED;
  }
  const int g = num_q_heads / num_kv_heads;
  const PrefillPlan plan = prefill_plan(num_seqs, num_q_heads, num_kv_heads, head_dim, block_size,
                                        max_blocks_per_seq, max_query_len);
  const int64_t grid = plan.col_blocks * plan.max_splits * num_seqs * num_kv_heads;
  if (grid > 0x7fffffff || plan.col_blocks > 0x7fffffff) {
    set_error("%lld workgroups exceed the grid limit", (long long)grid);
    return PA_ERR_UNSUPPORTED;
  }
  if (plan.ws_bytes && (!workspace || workspace_bytes < plan.ws_bytes)) {
    set_error("workspace of %zu bytes needed, %zu given", plan.ws_bytes, workspace_bytes);
    return PA_ERR_WORKSPACE;
  }
  PrefillAttnArgs a{};
  a.q = (const f16*)q;
  a.q_st = q_strides[0];
  a.q_sh = q_strides[1];
  a.k = (const f16*)k_cache;
  a.k_sb = k_strides[0];
  a.k_st = k_strides[1];
  a.k_sh = k_strides[2];
  a.v = (const f16*)v_cache;
  a.v_sb = v_strides[0];
  a.v_st = v_strides[1];
  a.v_sh = v_strides[2];
  a.bt = block_tables;
  a.bt_sb = bt_strides[0];
  a.bt_sk = bt_strides[1];
  a.lens = seq_lens;
  a.qstart = query_start_loc;
  a.out = (f16*)out;
  a.o_st = out_strides[0];
  a.o_sh = out_strides[1];
  a.num_seqs = num_seqs;
  a.num_tokens = num_tokens;
  a.hkv = num_kv_heads;
  a.g = g;
  a.bs = block_size;
  a.num_blocks = num_blocks;
  a.max_blocks = max_blocks_per_seq;
  a.col_blocks = (int)plan.col_blocks;
  a.col_groups = plan.col_groups;
  a.wave_groups = plan.wave_groups;
  a.scale_log2 = scale * kLog2e;
  a.split_tiles = (int)plan.split_tiles;
  a.max_splits = (int)plan.max_splits;
  a.cnt = plan.ws_bytes ? (int*)workspace : nullptr;
  a.recs = plan.ws_bytes ? (float*)((char*)workspace + plan.counter_bytes) : nullptr;
  return finish_launch(launch_prefill_attn(a, head_dim, (hipStream_t)stream));
}

int pa_rmsnorm_f16(const void* x, int64_t x_row_stride, const void* residual,
                   int64_t residual_row_stride, void* sum, int64_t sum_row_stride,
                   const void* weight, void* y, int64_t y_row_stride, int rows, int hidden,
                   float eps, void* stream) {
  clear_error();
  if (rows < 0 || hidden <= 0) {
    set_error("rows must be >= 0 and hidden > 0");
    return PA_ERR_ARG;
  }
  if (rows == 0) return PA_OK;
  if (!x || !weight || !y || (residual && !sum)) {
    set_error("null pointer argument");
    return PA_ERR_ARG;
  }
  if (x_row_stride < hidden || y_row_stride < hidden ||
      (residual && (residual_row_stride < hidden || sum_row_stride < hidden))) {
    set_error("row strides must be at least the hidden size");
    return PA_ERR_ARG;
  }
  return finish_launch(launch_rmsnorm((const f16*)x, x_row_stride, (const f16*)residual,
                                      residual_row_stride, (f16*)sum, sum_row_stride,
                                      (const f16*)weight, (f16*)y, y_row_stride, rows, hidden, eps,
                                      (hipStream_t)stream));
}

int pa_silu_mul_f16(const void* gate_up, int64_t gate_up_row_stride, void* out,
                    int64_t out_row_stride, int rows, int inter, void* stream) {
  clear_error();
  if (rows < 0 || inter <= 0) {
    set_error("rows must be >= 0 and inter > 0");
    return PA_ERR_ARG;
  }
  if (rows == 0) return PA_OK;
  if (!gate_up || !out) {
    set_error("null pointer argument");
    return PA_ERR_ARG;
  }
  if (gate_up_row_stride < 2 * (int64_t)inter || out_row_stride < inter) {
    set_error("gate_up rows need 2 * inter elements and out rows inter");
    return PA_ERR_ARG;
  }
  if ((int64_t)rows * inter > ((int64_t)1 << 38)) {
    set_error("rows * inter exceeds the launch grid");
    return PA_ERR_UNSUPPORTED;
  }
  const bool vec = inter % 8 == 0 && gate_up_row_stride % 8 == 0 && out_row_stride % 8 == 0 &&
                   aligned(gate_up, 16) && aligned(out, 16);
  return finish_launch(launch_silu_mul((const f16*)gate_up, gate_up_row_stride, (f16*)out,
                                       out_row_stride, rows, inter, vec, (hipStream_t)stream));
}

int pa_top2_f16(const void* logits, int64_t row_stride, int rows, int vocab, int64_t* index,
                float* top, void* stream) {
  clear_error();
  if (rows < 0 || vocab <= 0) {
    set_error("rows must be >= 0 and vocab > 0");
    return PA_ERR_ARG;
  }
  if (rows == 0) return PA_OK;
  if (!logits || !index || !top) {
    set_error("null pointer argument");
    return PA_ERR_ARG;
  }
  if (row_stride < vocab) {
    set_error("row stride must be at least the vocabulary size");
    return PA_ERR_ARG;
  }
  const bool vec = vocab % 8 == 0 && row_stride % 8 == 0 && aligned(logits, 16);
  return finish_launch(launch_top2((const f16*)logits, row_stride, rows, vocab, index, top, vec,
                                   (hipStream_t)stream));
}

}  // extern "C"
