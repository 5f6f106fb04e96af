// The projections of a decode step on gfx950: out = x . W^T for a handful of rows (one
// token per sequence, M <= 64 per row block) against a weight matrix that is read once
// per step, plus the residual add + RMSNorm that joins two projections.
//
// Reference behaviour: src/tinyserve/model.py:137-179, the decoder layer of the fused
// path: h = rms_norm(x); qkv = F.linear(h, W_qkv); ... x = x + F.linear(attn, W_o);
// h = rms_norm(x); [gate | up] = F.linear(h, W_gate_up); x = x + F.linear(silu(gate) * up,
// W_down). No reference kernel corresponds to these launches: they restate those PyTorch
// calls, with their roundings (each F.linear rounds its fp32 sums to the model dtype
// once; the residual add rounds the projection, then the sum; F.silu rounds, then the
// product with up rounds).
//
// rows_gemm. A decode step's projection is an HBM stream of W (2 bytes per weight, a
// few MB) against a few KB of x per row: the time is the stream's latency and rate, not
// arithmetic. Each wave owns NTW 16-row tiles of W over STEPS * 32 columns of K and all
// 64 rows of x's row block, issues every load of that share at once (W rows as
// v_mfma_f32_16x16x32 A operands, x as B operands) and only then multiplies: issued
// interleaved with the MFMAs, as the scheduler prefers, a wave keeps ~8 loads in flight
// and walks its share in several dependent round trips. KP waves of a workgroup split
// the workgroup's columns and add their partial tiles in LDS; KS workgroups split K and
// write fp32 partial sums, which the kernel that consumes the projection adds (the
// residual + RMSNorm below), so no workgroup waits for another.
//
// Every workgroup re-reads its rows of x from L2, NTW tiles of W per read: x in the
// natural row-major layout costs 16 rows x 64 bytes per operand load. Producers inside
// this file (the RMSNorm, the SiLU epilogue) can instead write x "operand-tiled": for row
// block mb, 32-column chunk c and 16-row tile mt, a 1 KB unit holds the 64 lanes' 16-byte
// operands in lane order, so each operand load is one contiguous 1 KB read.
//
//   element (m, k) of an operand-tiled [Mpad, K] matrix (Mpad = M rounded up to 64) is at
//   ((((m / 64) * (K / 32) + k / 32) * 4 + (m % 64) / 16) * 64 + ((k % 32) / 8) * 16 + m % 16) * 8 + k % 8
//
// Epilogues: kStore rounds each sum to T into a row-major [M, N] output (qkv); kPartial
// writes fp32 partial sums [KS][M][N] (o_proj, down_proj: their residual add is done by
// add_rms_norm); kSiluGateUp takes W = [gate rows; up rows] (2N rows), gives each wave a
// gate tile and the matching up tile, and writes act = silu(gate) * up operand-tiled
// [Mpad, N] (the down projection's x).
//
// add_rms_norm. One wave per row: v = round_T(x + round_T(sum of the KS partials, fixed
// order)) is the new residual stream (written back in place; x and xo may alias, since
// each element is loaded before it is stored), and h = RMSNorm(v) * w, rounded
// as rms_norm_rows rounds it, is written row-major or operand-tiled.
#include <cstdlib>

#include "common.h"

namespace ts {

typedef _Float16 r_f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 r_bf16x8 __attribute__((ext_vector_type(8)));
typedef float r_f32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Mfma16x32;
template <>
struct Mfma16x32<f16> {
  using V8 = r_f16x8;
  static __device__ __forceinline__ r_f32x4 mma(V8 a, V8 b, r_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma16x32<bf16> {
  using V8 = r_bf16x8;
  static __device__ __forceinline__ r_f32x4 mma(V8 a, V8 b, r_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

enum RowsEpilogue { kStore = 0, kPartial = 1, kSiluGateUp = 2 };

constexpr int kRowBlock = 64;  // rows of x per row block: four 16-row MFMA tiles

// Offset (in elements) of element (m, k) of an operand-tiled matrix with K columns.
__device__ __forceinline__ int64_t tiled_index(int m, int k, int K) {
  const int64_t unit = (static_cast<int64_t>(m / kRowBlock) * (K / 32) + k / 32) * 4 + (m % kRowBlock) / 16;
  return (unit * 64 + ((k % 32) / 8) * 16 + m % 16) * 8 + k % 8;
}

struct RowsArgs {
  const void* x;
  const void* w;
  void* out;       // kStore: T [M, N] (row stride os); kSiluGateUp: T operand-tiled [Mpad, N]
  float* partial;  // kPartial: fp32 [KS][M][N]
  int M, N, K;     // N: output columns (kSiluGateUp: W holds 2N rows)
  int ks;          // workgroups along K
  int kchunks;     // KP * STEPS * 32-column chunks per workgroup, walked one after another
  int64_t xs, ws, os;
};

// Lane l of a 16 x 32 operand holds row l % 16 and columns 8 (l / 16) .. + 7; the 16 x 16
// fp32 result holds column l % 16 (a row of x) and rows 4 (l / 16) .. + 3 (rows of W).
template <typename T, int KP, int NTW, int STEPS, bool XT, int EPI>
__global__ __launch_bounds__(KP * kWave) void rows_gemm_kernel(const RowsArgs a) {
  using V8 = typename Mfma16x32<T>::V8;
  static_assert(EPI != kSiluGateUp || NTW == 2, "SiLU epilogue: one gate and one up tile per wave");
  constexpr int BN = 16 * NTW;  // W rows per workgroup
  constexpr int RED = BN + 1;   // padded row of the part sums
  __shared__ float red[KP > 1 ? KP * kRowBlock * RED : 1];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int kp = tid / kWave;
  const int r16 = lane & 15;
  const int kq = (lane >> 4) * 8;
  const int mb = blockIdx.y;
  // Output columns of the workgroup: n0 .. n0 + BN - 1 (SiLU: n0 .. n0 + 15 of gate and
  // of up).
  const int n0 = blockIdx.x * (EPI == kSiluGateUp ? 16 : BN);
  constexpr int CH = KP * STEPS * 32;  // columns of one chunk
  const T* __restrict__ xg = static_cast<const T*>(a.x);
  const T* __restrict__ wg = static_cast<const T*>(a.w);

  // W row of tile t for this lane.
  auto w_row = [&](int t) {
    if constexpr (EPI == kSiluGateUp) return (t == 0 ? n0 : a.N + n0) + r16;
    else return n0 + t * 16 + r16;
  };
  // x row of MFMA tile mt for this lane (rows past M read row M - 1: finite, never
  // stored).
  int xrow[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) xrow[mt] = min(mb * kRowBlock + mt * 16 + r16, a.M - 1);

  r_f32x4 acc[NTW][4];
#pragma unroll
  for (int t = 0; t < NTW; ++t)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) acc[t][mt] = r_f32x4{0.f, 0.f, 0.f, 0.f};

  for (int c = 0; c < a.kchunks; ++c) {
    const int k0 = (blockIdx.z * a.kchunks + c) * CH + kp * (STEPS * 32);  // this wave's columns
    V8 wv[STEPS][NTW], xv[STEPS][4];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int k = k0 + s * 32;
#pragma unroll
      for (int t = 0; t < NTW; ++t)
        wv[s][t] = *reinterpret_cast<const V8*>(wg + static_cast<int64_t>(w_row(t)) * a.ws + k + kq);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        if constexpr (XT) {
          const int64_t unit = (static_cast<int64_t>(mb) * (a.K / 32) + k / 32) * 4 + mt;
          xv[s][mt] = *reinterpret_cast<const V8*>(xg + unit * 512 + lane * 8);
        } else {
          xv[s][mt] = *reinterpret_cast<const V8*>(xg + static_cast<int64_t>(xrow[mt]) * a.xs + k + kq);
        }
      }
    }
    // Every load of the chunk is issued before the first multiply.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < STEPS; ++s)
#pragma unroll
      for (int t = 0; t < NTW; ++t)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) acc[t][mt] = Mfma16x32<T>::mma(wv[s][t], xv[s][mt], acc[t][mt]);
  }

  // Sum of the KP waves' parts of element (m, j), j < BN the workgroup's W row.
  if constexpr (KP > 1) {
#pragma unroll
    for (int t = 0; t < NTW; ++t)
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          red[(kp * kRowBlock + mt * 16 + r16) * RED + t * 16 + (lane >> 4) * 4 + i] = acc[t][mt][i];
    __syncthreads();
  }
  auto total = [&](int m, int j) {
    float v = 0.f;
#pragma unroll
    for (int p = 0; p < KP; ++p) v += red[(p * kRowBlock + m) * RED + j];
    return v;
  };

  if constexpr (KP > 1 && EPI == kSiluGateUp) {
    // One output element per thread at a time (consecutive threads, consecutive
    // columns): the SiLU's exp and roundings are spread over every thread. Rows past M
    // are written as zeros: the tiled output is read whole.
    for (int u = tid; u < kRowBlock * 16; u += KP * kWave) {
      const int m = u / 16, j = u % 16;
      const int row = mb * kRowBlock + m;
      float v = 0.f;
      if (row < a.M) {
        const float g = to_f32(from_f32<T>(total(m, j)));
        const float up = to_f32(from_f32<T>(total(m, 16 + j)));
        v = to_f32(from_f32<T>(g / (1.0f + expf(-g)))) * up;
      }
      static_cast<T*>(a.out)[tiled_index(row, n0 + j, a.N)] = from_f32<T>(v);
    }
  } else if constexpr (KP > 1) {
    // Thread u handles 8 consecutive columns of one row: 16-byte stores.
    constexpr int GROUPS = BN / 8;
    for (int u = tid; u < kRowBlock * GROUPS; u += KP * kWave) {
      const int m = u / GROUPS, j0 = (u % GROUPS) * 8;
      const int row = mb * kRowBlock + m;
      if (row >= a.M) continue;
      if constexpr (EPI == kStore) {
        Pack16<T> y;
#pragma unroll
        for (int e = 0; e < 8; ++e) y.v[e] = from_f32<T>(total(m, j0 + e));
        store16(static_cast<T*>(a.out) + row * a.os + n0 + j0, y);
      } else {
        float* p = a.partial + (static_cast<int64_t>(blockIdx.z) * a.M + row) * a.N + n0 + j0;
        *reinterpret_cast<r_f32x4*>(p) = r_f32x4{total(m, j0), total(m, j0 + 1), total(m, j0 + 2), total(m, j0 + 3)};
        *reinterpret_cast<r_f32x4*>(p + 4) =
            r_f32x4{total(m, j0 + 4), total(m, j0 + 5), total(m, j0 + 6), total(m, j0 + 7)};
      }
    }
  } else {
    // One wave: each lane writes its own results (4 W rows of one x row per tile).
    if constexpr (EPI == kSiluGateUp) {
      // Tiles 0 (gate) and 1 (up) hold the same (row, column) positions in each lane.
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int row = mb * kRowBlock + mt * 16 + r16;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v = 0.f;  // rows past M: zeros (the tiled output is read whole)
          if (row < a.M) {
            const float g = to_f32(from_f32<T>(acc[0][mt][i]));
            const float up = to_f32(from_f32<T>(acc[1][mt][i]));
            v = to_f32(from_f32<T>(g / (1.0f + expf(-g)))) * up;
          }
          static_cast<T*>(a.out)[tiled_index(row, n0 + (lane >> 4) * 4 + i, a.N)] = from_f32<T>(v);
        }
      }
      return;
    }
#pragma unroll
    for (int t = 0; t < NTW; ++t)
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int row = mb * kRowBlock + mt * 16 + r16;
        if (row >= a.M) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int n = n0 + t * 16 + (lane >> 4) * 4 + i;
          if constexpr (EPI == kStore) static_cast<T*>(a.out)[row * a.os + n] = from_f32<T>(acc[t][mt][i]);
          else a.partial[(static_cast<int64_t>(blockIdx.z) * a.M + row) * a.N + n] = acc[t][mt][i];
        }
      }
  }
}

// ---- launch shapes -----------------------------------------------------------------------
struct RowsPlan {
  int kp, ntw, steps, ks, kchunks;
};

// Candidate (KP, NTW, STEPS) per epilogue, in order of preference; KS then follows from
// K. Measured on MI355X at Qwen3-0.6B shapes with 64 rows and W read cold from HBM
// (fp16, graph replay, us per launch; the library GEMM in brackets):
//   qkv     N 4096, K 1024, kStore, x tiled:         8 waves x 1 tile x 4 steps, KS 1: 5.7 (11.5)
//   o_proj  N 1024, K 2048, kPartial, x row-major:   4 waves x 2 tiles x 2 steps, KS 8: 4.7 (10.6)
//   gate_up N 2 x 3072, K 1024, SiLU, x tiled:       8 waves x 2 tiles x 4 steps, KS 1: 7.6 (11.7)
//   down    N 1024, K 3072, kPartial, x tiled:       8 waves x 2 tiles x 2 steps, KS 6: 5.1 (9.3)
// Across these, ~256 workgroups (one per CU) with each wave's loads in one round trip
// was the best shape; fewer, larger workgroups or more K splits were slower.
constexpr int kMaxSplits = 16;

static bool plan_rows(int M, int N, int K, int epi, RowsPlan* p) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 32) return false;
  struct Cand {
    int kp, ntw, steps;
  };
  static const Cand kStoreC[] = {{8, 1, 4}, {8, 1, 2}, {4, 1, 2}, {4, 1, 1}, {2, 1, 1}, {1, 1, 1}};
  static const Cand kPartC[] = {{8, 2, 2}, {4, 2, 2}, {8, 1, 2}, {4, 1, 2}, {4, 1, 1}, {2, 1, 1}, {1, 1, 1}};
  static const Cand kSiluC[] = {{8, 2, 4}, {8, 2, 2}, {4, 2, 2}, {4, 2, 1}, {2, 2, 1}, {1, 2, 1}};
  const Cand* cands = epi == kStore ? kStoreC : epi == kPartial ? kPartC : kSiluC;
  const int n = epi == kStore ? 6 : epi == kPartial ? 7 : 6;
  const int64_t mblocks = (M + kRowBlock - 1) / kRowBlock;
  const int want = compute_units();
  bool found = false;
  int64_t best_dist = 0;
  for (int i = 0; i < n; ++i) {
    const Cand& c = cands[i];
    const int ch = c.kp * c.steps * 32;
    const int bn = epi == kSiluGateUp ? 16 : 16 * c.ntw;
    if (K % ch || N % bn) continue;
    const int chunks = K / ch;
    int ks = 1;
    if (epi == kPartial) {
      // The divisor of the chunk count (at most kMaxSplits) that brings the grid closest
      // to the chip's CUs (K = 3072 in 512-column chunks: 6 splits).
      const int64_t tiles = N / bn * mblocks;
      for (int d = 2; d <= kMaxSplits && d <= chunks; ++d)
        if (chunks % d == 0 && std::abs(tiles * d - want) < std::abs(tiles * ks - want)) ks = d;
    }
    const int64_t grid = N / bn * mblocks * ks;
    const int64_t dist = std::abs(grid - want);
    // The first candidate whose grid lands within [3/4, 2] x the CUs; otherwise the one
    // nearest to the CU count.
    if (grid * 4 >= want * 3 && grid <= 2 * want) {
      *p = RowsPlan{c.kp, c.ntw, c.steps, ks, chunks / ks};
      return true;
    }
    if (!found || dist < best_dist) {
      found = true;
      best_dist = dist;
      *p = RowsPlan{c.kp, c.ntw, c.steps, ks, chunks / ks};
    }
  }
  return found;
}

template <typename T, int KP, int NTW, int STEPS, int EPI>
static int launch_rows(const RowsArgs& a, bool xt, hipStream_t st) {
  const int bn = EPI == kSiluGateUp ? 16 : 16 * NTW;
  const dim3 grid(a.N / bn, (a.M + kRowBlock - 1) / kRowBlock, a.ks);
  if (xt) hipLaunchKernelGGL((rows_gemm_kernel<T, KP, NTW, STEPS, true, EPI>), grid, dim3(KP * kWave), 0, st, a);
  else hipLaunchKernelGGL((rows_gemm_kernel<T, KP, NTW, STEPS, false, EPI>), grid, dim3(KP * kWave), 0, st, a);
  return launch_status();
}

template <typename T, int EPI>
static int dispatch_rows(const RowsArgs& a, const RowsPlan& p, bool xt, hipStream_t st) {
#define TS_ROWS(KP, NTW, S)                                      \
  if (p.kp == KP && p.ntw == NTW && p.steps == S) return launch_rows<T, KP, NTW, S, EPI>(a, xt, st);
  if constexpr (EPI == kStore) {
    TS_ROWS(8, 1, 4) TS_ROWS(8, 1, 2) TS_ROWS(4, 1, 2) TS_ROWS(4, 1, 1) TS_ROWS(2, 1, 1) TS_ROWS(1, 1, 1)
  } else if constexpr (EPI == kPartial) {
    TS_ROWS(8, 2, 2) TS_ROWS(4, 2, 2) TS_ROWS(8, 1, 2) TS_ROWS(4, 1, 2) TS_ROWS(4, 1, 1) TS_ROWS(2, 1, 1)
    TS_ROWS(1, 1, 1)
  } else {
    TS_ROWS(8, 2, 4) TS_ROWS(8, 2, 2) TS_ROWS(4, 2, 2) TS_ROWS(4, 2, 1) TS_ROWS(2, 2, 1) TS_ROWS(1, 2, 1)
  }
#undef TS_ROWS
  return TS_EUNSUPPORTED;
}

// ---- add_rms_norm -----------------------------------------------------------------------
// One wave per row; lane l holds 8-element chunks l, l + 64, ... (CPL of them).
template <typename T, int CPL>
__global__ __launch_bounds__(64) void add_rms_norm_kernel(const T* x, const float* __restrict__ part,
                                                           int ks, const T* __restrict__ w, T* xo,
                                                           T* __restrict__ h, bool h_tiled, int M, int rows,
                                                           int N, int64_t xs, int64_t xos, int64_t hs,
                                                           float eps) {
  const int lane = threadIdx.x & (kWave - 1);
  // One wave per workgroup: a decode step's few rows land on as many CUs, each pulling
  // only its row's partials through its own L1.
  const int row = blockIdx.x;
  if (row >= rows) return;
  if (row >= M) {
    // Padding rows of an operand-tiled output (read whole by the projection): zeros.
    for (int i = lane * 8; i < N; i += kWave * 8) {
      Pack16<T> z;
      z.raw = u32x4{0, 0, 0, 0};
      store16(h + tiled_index(row, i, N), z);
    }
    return;
  }
  Pack16<T> xv[CPL], wv[CPL];
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int i = (k * kWave + lane) * 8;
    if (i < N) {
      xv[k] = load16(x + row * xs + i);
      wv[k] = load16(w + i);
    }
  }
  if (ks > 0) {
    // The residual stream as model.py:172,179 computes it: the projection (the sum of
    // its partials in z order) is rounded to T, then x + it is rounded again. The partials are loaded ZG at a time, every load of a group issued before the
    // first add (ZG * CPL * 8 floats of registers): one round trip per group instead of
    // one per partial.
    constexpr int ZG = 16 / CPL > 0 ? 16 / CPL : 1;
    float s[CPL][8];
#pragma unroll
    for (int k = 0; k < CPL; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) s[k][e] = 0.f;
    for (int z0 = 0; z0 < ks; z0 += ZG) {
      r_f32x4 pv[ZG][CPL][2];
#pragma unroll
      for (int z = 0; z < ZG; ++z) {
        if (z0 + z < ks) {
#pragma unroll
          for (int k = 0; k < CPL; ++k) {
            const int i = (k * kWave + lane) * 8;
            if (i < N) {
              const float* p = part + (static_cast<int64_t>(z0 + z) * M + row) * N + i;
              pv[z][k][0] = *reinterpret_cast<const r_f32x4*>(p);
              pv[z][k][1] = *reinterpret_cast<const r_f32x4*>(p + 4);
            }
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int z = 0; z < ZG; ++z) {
        if (z0 + z < ks) {
#pragma unroll
          for (int k = 0; k < CPL; ++k)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              s[k][e] += pv[z][k][0][e];
              s[k][4 + e] += pv[z][k][1][e];
            }
        }
      }
    }
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      const int i = (k * kWave + lane) * 8;
      if (i >= N) continue;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        xv[k].v[e] = from_f32<T>(to_f32(from_f32<T>(s[k][e])) + to_f32(xv[k].v[e]));
      store16(xo + row * xos + i, xv[k]);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int i = (k * kWave + lane) * 8;
    if (i < N) {
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(to_f32(xv[k].v[e]), to_f32(xv[k].v[e]), ss);
    }
  }
  ss = group_sum<kWave>(ss);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(N) + eps);
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int i = (k * kWave + lane) * 8;
    if (i >= N) continue;
    Pack16<T> y;
#pragma unroll
    for (int e = 0; e < 8; ++e) y.v[e] = norm_scale(xv[k].v[e], r, wv[k].v[e]);
    store16(h + (h_tiled ? tiled_index(row, i, N) : row * hs + i), y);
  }
}

template <typename T>
static int launch_add_rms(const void* x, int64_t xs, const float* part, int ks, const void* w, void* xo,
                          int64_t xos, void* h, bool h_tiled, int64_t hs, int M, int N, float eps,
                          hipStream_t st) {
  const int cpl = (N + kWave * 8 - 1) / (kWave * 8);
  const int rows = h_tiled ? (M + kRowBlock - 1) / kRowBlock * kRowBlock : M;
  const dim3 grid(rows), block(kWave);
  const T* xp = static_cast<const T*>(x);
  const T* wp = static_cast<const T*>(w);
  T* xop = static_cast<T*>(xo);
  T* hp = static_cast<T*>(h);
#define TS_ARN(C) \
  hipLaunchKernelGGL((add_rms_norm_kernel<T, C>), grid, block, 0, st, xp, part, ks, wp, xop, hp, h_tiled, M, rows, N, xs, xos, hs, eps)
  if (cpl <= 1) TS_ARN(1);
  else if (cpl <= 2) TS_ARN(2);
  else if (cpl <= 4) TS_ARN(4);
  else if (cpl <= 8) TS_ARN(8);
  else return TS_EUNSUPPORTED;
#undef TS_ARN
  return launch_status();
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace ts

using namespace ts;

extern "C" int ts_rows_gemm_plan(int M, int N, int K, int epilogue, int* out) {
  if (!out || epilogue < kStore || epilogue > kSiluGateUp) return TS_EINVAL;
  RowsPlan p;
  if (!plan_rows(M, N, K, epilogue, &p)) return TS_EUNSUPPORTED;
  out[0] = p.kp;
  out[1] = p.ntw;
  out[2] = p.steps;
  out[3] = p.ks;
  out[4] = p.kchunks;
  return 0;
}

extern "C" int ts_rows_gemm(const void* x, int x_tiled, int64_t x_stride, const void* w, int64_t w_stride,
                            void* out, int64_t o_stride, float* partial, int64_t partial_floats, int M,
                            int N, int K, int epilogue, int dtype, void* stream) {
  if (M < 0 || N <= 0 || K <= 0 || epilogue < kStore || epilogue > kSiluGateUp) return TS_EINVAL;
  if (!x || !w || w_stride < K || (!x_tiled && x_stride < K) || (x_tiled && K % 32)) return TS_EINVAL;
  if (epilogue == kStore && (!out || o_stride < N)) return TS_EINVAL;
  if (epilogue == kSiluGateUp && (!out || N % 32)) return TS_EINVAL;  // out is operand-tiled
  if (M == 0) return 0;
  if (dtype != TS_F16 && dtype != TS_BF16) return TS_EUNSUPPORTED;
  // 16-byte operand loads and stores.
  if (!aligned16(x) || !aligned16(w) || (out && !aligned16(out)) || (partial && !aligned16(partial)) ||
      w_stride % 8 || (!x_tiled && x_stride % 8) || (epilogue == kStore && o_stride % 8))
    return TS_EUNSUPPORTED;
  RowsPlan p;
  if (!plan_rows(M, N, K, epilogue, &p)) return TS_EUNSUPPORTED;
  if (epilogue == kPartial && (!partial || partial_floats < static_cast<int64_t>(p.ks) * M * N))
    return TS_EINVAL;
  RowsArgs a{x, w, out, partial, M, N, K, p.ks, p.kchunks, x_stride, w_stride, o_stride};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool xt = x_tiled != 0;
  switch (epilogue) {
    case kStore:
      return dtype == TS_F16 ? dispatch_rows<f16, kStore>(a, p, xt, st) : dispatch_rows<bf16, kStore>(a, p, xt, st);
    case kPartial:
      return dtype == TS_F16 ? dispatch_rows<f16, kPartial>(a, p, xt, st) : dispatch_rows<bf16, kPartial>(a, p, xt, st);
    default:
      return dtype == TS_F16 ? dispatch_rows<f16, kSiluGateUp>(a, p, xt, st)
                             : dispatch_rows<bf16, kSiluGateUp>(a, p, xt, st);
  }
}

extern "C" int ts_add_rms_norm(const void* x, int64_t x_stride, const float* partial, int ks, const void* w,
                               void* x_out, int64_t xo_stride, void* h, int h_tiled, int64_t h_stride, int M,
                               int N, float eps, int dtype, void* stream) {
  if (M < 0 || N <= 0 || ks < 0 || !x || !w || !h || x_stride < N) return TS_EINVAL;
  if (ks > 0 && (!partial || !x_out || xo_stride < N)) return TS_EINVAL;
  if (!h_tiled && h_stride < N) return TS_EINVAL;
  if (M == 0) return 0;
  if (dtype != TS_F16 && dtype != TS_BF16) return TS_EUNSUPPORTED;
  if (N % 8 || x_stride % 8 || (ks > 0 && xo_stride % 8) || (!h_tiled && h_stride % 8) ||
      (h_tiled && N % 32) || !aligned16(x) || !aligned16(w) || !aligned16(h) ||
      (ks > 0 && (!aligned16(partial) || !aligned16(x_out))))
    return TS_EUNSUPPORTED;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return dtype == TS_F16 ? launch_add_rms<f16>(x, x_stride, partial, ks, w, x_out, xo_stride, h, h_tiled != 0,
                                               h_stride, M, N, eps, st)
                         : launch_add_rms<bf16>(x, x_stride, partial, ks, w, x_out, xo_stride, h, h_tiled != 0,
                                                h_stride, M, N, eps, st);
}
