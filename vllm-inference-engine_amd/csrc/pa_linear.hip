// Decode-step linear layers for gfx950: Y = X W^T with the decoder layer's
// epilogues, for the few hundred rows (one per sequence) a decode step has.
//
// At these sizes the projections are bound by streaming the weights (1.6-17 MB
// per matrix for a 0.5B model against 0.2-1.2 MB of activations), and a
// library GEMM tiled for large M spreads a matrix over too few workgroups with
// too little in flight. This kernel:
//   * gives each workgroup 16 x NTW weight rows (output columns) and all 128
//     rows of an M tile; its four wavefronts take every fourth K step each
//     over the whole tile, so each operand byte is loaded once per
//     workgroup, and their tiles are summed through LDS in a fixed order;
//   * splits K over workgroups until about one workgroup per CU is busy; the
//     last workgroup of a tile to finish sums the partial tiles in split order
//     (the same bits whichever finishes last) and applies the epilogue;
//   * forms Y^T tiles with v_mfma_f32_16x16x32_f16, weight rows as the A
//     operand and X rows as the B operand, so both operands are read 16 bytes
//     at a time straight along K from memory, without LDS staging;
//   * keeps two K steps of loads in flight per wavefront. Loads past the
//     split's end go through a buffer resource of extent 0, which returns
//     zeros without touching memory, so the loop has no branches.
// Epilogues (fp32 accumulation, roundings of the unfused decoder layer):
//   kLinStore:  Y = fp16(acc + bias)        nn.Linear (bias optional)
//   kLinAdd:    Y = fp16(Y + acc)            torch.addmm_ into Y
//   kLinSwiglu: weight rows [0, N) are the gate projection and [N, 2N) the up
//               projection; Y = fp16(fp16(silu(fp16(acc_gate))) * fp16(acc_up))
#include "pa_tiles.h"

namespace pa {
using namespace tiles;

namespace {

template <int NTW, int EPI>
__global__ __launch_bounds__(256) void linear_kernel(LinearArgs a) {
  constexpr int MTW = 8;       // X tiles of 16 rows: the 128-row M tile
  constexpr int TQ = 2 * NTW;  // f32x4 accumulators per lane after the wavefront reduction
  __shared__ f32x4 s_red[4][NTW * MTW][64];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int i = lane & 15;
  const int g = lane >> 4;
  const int S = a.splits;
  const int tile = blockIdx.x / S;
  const int s = blockIdx.x - tile * S;
  const int nt = tile % a.n_tiles;
  const int mt = tile / a.n_tiles;
  const int KS = a.K >> 5;  // K steps of 32
  const int st0 = (int)((int64_t)s * KS / S);
  const int st1 = (int)((int64_t)(s + 1) * KS / S);

  // Byte offsets of this lane's 16-byte piece of each operand row at k = 0.
  // Rows past the end re-read the last row; their results are never stored.
  uint32_t xo[MTW], wo[NTW];
#pragma unroll
  for (int u = 0; u < MTW; ++u) {
    int m = mt * 128 + 16 * u + i;
    m = m < a.M ? m : a.M - 1;
    xo[u] = (uint32_t)(2 * ((int64_t)m * a.xs + 8 * g));
  }
#pragma unroll
  for (int t = 0; t < NTW; ++t) {
    int n;
    if constexpr (EPI == kLinSwiglu) {
      constexpr int H = NTW / 2;
      int c = nt * (16 * H) + 16 * (t % H) + i;
      c = c < a.N ? c : a.N - 1;
      n = t < H ? c : a.N + c;
    } else {
      n = nt * (16 * NTW) + 16 * t + i;
      n = n < a.N ? n : a.N - 1;
    }
    wo[t] = (uint32_t)(2 * ((int64_t)n * a.wsr + 8 * g));
  }
  // A step past the split's end reads through resources of extent 0, whose
  // loads return zeros without touching memory: the choice is a scalar one,
  // and the per-lane offsets stay fixed (the step enters as the scalar offset).
  const auto xr = tile_rsrc(a.x, a.x_bytes);
  const auto wr = tile_rsrc(a.w, a.w_bytes);
  const auto xr0 = tile_rsrc(a.x, 0);
  const auto wr0 = tile_rsrc(a.w, 0);

  // Each wavefront accumulates the whole tile over every fourth K step of the
  // split (so every operand byte is loaded once per workgroup).
  f32x4 acc[NTW][MTW];
#pragma unroll
  for (int t = 0; t < NTW; ++t)
#pragma unroll
    for (int u = 0; u < MTW; ++u) acc[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Buffers hold raw 16-byte pieces (u32x4, cast at the product): as fp16
  // vectors the compiler would splice new loads into a merged vector with bit
  // inserts that wait for the loads there.
  u32x4 w0[NTW], x0[MTW], w1[NTW], x1[MTW];
  auto load = [&](u32x4 (&wv)[NTW], u32x4 (&xv)[MTW], int st) {
    const bool live = st < st1;
    const auto wrs = live ? wr : wr0;
    const auto xrs = live ? xr : xr0;
    const int kb = live ? st << 6 : 0;  // 32 halves
#pragma unroll
    for (int t = 0; t < NTW; ++t)  // weights are read once: non-temporal
      wv[t] = __builtin_amdgcn_raw_buffer_load_b128(wrs, wo[t], kb, 3);
#pragma unroll
    for (int u = 0; u < MTW; ++u)  // activations are shared by every column tile: cached
      xv[u] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xo[u], kb, 0);
  };
  auto mma = [&](const u32x4 (&wv)[NTW], const u32x4 (&xv)[MTW]) {
#pragma unroll
    for (int t = 0; t < NTW; ++t)
#pragma unroll
      for (int u = 0; u < MTW; ++u)
        acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, wv[t]),
                                                           __builtin_bit_cast(f16x8, xv[u]),
                                                           acc[t][u], 0, 0, 0);
  };

  // The phases are kept in this order (the scheduler would otherwise mix the
  // next step's loads into the products and drain every load each iteration):
  // the products of one buffer run while the other buffer's loads are in flight.
  load(w0, x0, st0 + wave);
  __builtin_amdgcn_sched_barrier(0);
  load(w1, x1, st0 + wave + 4);
  __builtin_amdgcn_sched_barrier(0);
  for (int st = st0 + wave; st < st1; st += 8) {
    mma(w0, x0);
    __builtin_amdgcn_sched_barrier(0);
    load(w0, x0, st + 8);
    __builtin_amdgcn_sched_barrier(0);
    mma(w1, x1);
    __builtin_amdgcn_sched_barrier(0);
    load(w1, x1, st + 12);
    __builtin_amdgcn_sched_barrier(0);
  }

  // Sum the four wavefronts' tiles in wavefront order; wavefront w keeps rows
  // [32 w, 32 w + 32) of the tile: r[t][v] is X tile 2 w + v.
#pragma unroll
  for (int t = 0; t < NTW; ++t)
#pragma unroll
    for (int u = 0; u < MTW; ++u) s_red[wave][t * MTW + u][lane] = acc[t][u];
  __syncthreads();
  f32x4 r[NTW][2];
#pragma unroll
  for (int t = 0; t < NTW; ++t)
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const int q = t * MTW + 2 * wave + v;
      r[t][v] = ((s_red[0][q][lane] + s_red[1][q][lane]) + s_red[2][q][lane]) + s_red[3][q][lane];
    }

  if (S > 1) {
    // Publish this split's tile in lane order (16-byte device-coherent
    // stores), count one arrival; the last arrival sums all splits in order.
    __shared__ int s_last;
    const auto pr = tile_rsrc(a.part, a.part_bytes);
    const int base = (tile * S + s) * TQ * 256;
#pragma unroll
    for (int t = 0; t < NTW; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u)
        store_coherent16(pr, 16 * (base + (t * 2 + u) * 256 + tid), r[t][u]);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
      const int old =
          __hip_atomic_fetch_add(a.cnt + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = old == S - 1;
    }
    __syncthreads();
    if (!s_last) return;
#pragma unroll
    for (int t = 0; t < NTW; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u) r[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int sp = 0; sp < S; ++sp) {
      const int rb = (tile * S + sp) * TQ * 256;
#pragma unroll
      for (int t = 0; t < NTW; ++t)
#pragma unroll
        for (int u = 0; u < 2; ++u)
          r[t][u] += load_coherent16(pr, 16 * (rb + (t * 2 + u) * 256 + tid));
    }
    if (tid == 0) __hip_atomic_store(a.cnt + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // Lane (i, g) of accumulator (t, u) holds Y[m][n .. n + 3] with
  // m = 16 u + i and n = 16 t + 4 g within the tile.
  constexpr int TO = EPI == kLinSwiglu ? NTW / 2 : NTW;  // output column groups of 16
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int m = mt * 128 + wave * 32 + 16 * u + i;
    if (m >= a.M) continue;
#pragma unroll
    for (int t = 0; t < TO; ++t) {
      const int n = nt * (16 * TO) + 16 * t + 4 * g;
      if (n >= a.N) continue;
      f16* yp = a.y + (int64_t)m * a.ys + n;
      f16x4 o;
      if constexpr (EPI == kLinSwiglu) {
        const f32x4 gt = r[t][u], up = r[t + TO][u];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float gf = (float)(f16)gt[e];
          const f16 sl = (f16)(gf / (1.f + expf(-gf)));
          o[e] = (f16)((float)sl * (float)(f16)up[e]);
        }
      } else {
        f32x4 v = r[t][u];
        if constexpr (EPI == kLinAdd) {
          const f16x4 old = *reinterpret_cast<const f16x4*>(yp);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] += (float)old[e];
        } else {
          if (a.bias) {
            const f16x4 bv = *reinterpret_cast<const f16x4*>(a.bias + n);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] += (float)bv[e];
          }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = (f16)v[e];
      }
      *reinterpret_cast<f16x4*>(yp) = o;
    }
  }
}

template <int EPI>
hipError_t launch_linear_e(const LinearArgs& a, hipStream_t s) {
  const int m_tiles = (a.M + 127) / 128;
  const dim3 grid((unsigned)(a.n_tiles * m_tiles * a.splits));
  hipLaunchKernelGGL((linear_kernel<kLinearNtw, EPI>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_linear(const LinearArgs& a, int epilogue, hipStream_t s) {
  switch (epilogue) {
    case kLinStore: return launch_linear_e<kLinStore>(a, s);
    case kLinAdd: return launch_linear_e<kLinAdd>(a, s);
    case kLinSwiglu: return launch_linear_e<kLinSwiglu>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace pa
