// Varlen causal prefill attention over the paged KV cache, on gfx950 MFMA.
//
// Reference behaviour: src/tinyserve/triton_prefill.py:50-125 (one program per
// (sequence, query tile, kv head), keys walked in chunks from position 0 to the tile's
// last query position, online softmax, P rounded to the value dtype before P.V) and
// src/tinyserve/attention.py:62-111 for the math it must equal.
//
// Work decomposition. A workgroup of 4 wave64s owns one kv head of one sequence and
// 32 * QB consecutive queries of HG of the kv head's query heads (HG * QB = 4): wave w
// takes query head hg = w % HG and the 32 queries of block qb = w / HG. All four
// waves share each 64-key tile of K and V, which the workgroup gathers from the paged
// cache (slot = table[pos / bs] * bs + pos % bs) into LDS once.
//
// MFMA formulation (v_mfma_f32_32x32x16_{f16,bf16}). Scores are computed transposed,
// S^T[key, query] = K . Q^T, with K as the A operand (from LDS, 16 contiguous bytes of a
// key row per lane) and Q^T as the B operand (held in registers for the whole kernel).
// In the 32x32 accumulator layout lane l holds column l % 32 -- one query -- and rows
// (keys) 8j + 4(l / 32) + i at item 4j + i, so each lane owns 16 of its query's scores
// per 32 keys: the softmax max/sum are in-lane plus one exchange between the lane halves.
// The output is accumulated transposed too, O^T[d, query] += V^T . P^T: P^T is the B
// operand straight from the score registers (lane half h supplies keys
// {4h..4h+3, 8+4h..8+4h+3} of each 16-key chunk, an order the A operand repeats), and
// V^T is the A operand, read from a transposed copy of the V tile in LDS (key-major per
// d row, 4-key groups XOR-swizzled by d to spread the reads over the banks).
#include <type_traits>

#include "common.h"

namespace ts {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <typename T>
struct Mfma;
template <>
struct Mfma<f16> {
  using V8 = f16x8;
  static __device__ __forceinline__ f32x16 mma(V8 a, V8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma<bf16> {
  using V8 = bf16x8;
  static __device__ __forceinline__ f32x16 mma(V8 a, V8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

struct PrefillArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  const int32_t* bt;
  const int32_t* q_starts;
  const int32_t* q_lens;
  const int32_t* ctx_lens;
  int R;
  int group;
  int hchunks;  // group / HG
  int lbs;
  int n_qtiles;
  int64_t q_st, q_sh, o_st, o_sh, k_ss, k_sh, bt_s;
  float scale_log2;
};

constexpr int kBN = 64;        // keys per LDS tile
constexpr int kThreads = 256;  // 4 waves

template <typename T, int D>
struct PrefillShape {
  static constexpr int kCH = D / 8;                  // 16-byte units of a row
  static constexpr int kKPT = kBN * kCH / kThreads;  // keys staged per thread
  static constexpr int kNKG = kBN / kKPT;            // key groups (threads per row part)
  static_assert(kKPT >= 2 && kKPT <= 4, "D in {64, 128}");
};

// LDS layouts (bank-conflict free for the MFMA operand reads with 32 or 64 banks, and for
// the staging writes with 32 banks; modelled per access pattern before use).
// K tile: row `key` of D elements, its 16-byte units XOR-swizzled by the key.
template <int CH>
__device__ __forceinline__ int k_unit(int key, int unit) {
  return unit ^ ((key ^ (key >> 3)) & (CH - 1));
}
__device__ __forceinline__ int vt_swz(int d) { return (d ^ (d >> 3)) & 7; }

// Column of key `key` (0..63) in row d of the transposed V tile. The 16-key chunk c0 is
// stored as two 8-key units, unit 2 c0 + h holding keys {16c0 + 4h .. +3, 16c0 + 8 + 4h
// .. +3} -- exactly the 8 k-values lane half h supplies to an MFMA operand -- so each
// operand is one 16-byte read; units are XOR-swizzled by d.
__device__ __forceinline__ int vt_col(int key, int d) {
  const int unit = ((key >> 4) << 1) | ((key >> 2) & 1);
  const int within = (((key >> 3) & 1) << 2) | (key & 3);
  return ((unit ^ vt_swz(d)) << 3) | within;
}

template <typename T, int D, int HG, int QB>
__global__ __launch_bounds__(kThreads, 2) void prefill_mfma_kernel(const PrefillArgs a) {
  using Sh = PrefillShape<T, D>;
  using V8 = typename Mfma<T>::V8;
  constexpr int CH = Sh::kCH, KPT = Sh::kKPT, NKG = Sh::kNKG;
  constexpr int BQ = 32 * QB;
  constexpr int DT = D / 32;  // 32-row output tiles
  constexpr int KC = D / 16;  // 16-wide MFMA k-chunks of the head dim
  // bf16 keeps 8 significant bits: P rounded once would move outputs by up to ~1e-2
  // against the fp32 reference, so P is carried as hi + lo bf16 parts (about 16 bits)
  // and P.V takes two MFMAs. fp16's 11 bits meet the tolerance with one.
  constexpr bool kSplitP = std::is_same_v<T, bf16>;

  __shared__ __attribute__((aligned(16))) T k_lds[kBN * D];
  __shared__ __attribute__((aligned(16))) T vt_lds[D * kBN];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;  // this lane's query within the wave's 32
  const int half = lane >> 5;

  const int tile_rev = blockIdx.x / a.R;
  const int r = blockIdx.x - tile_rev * a.R;
  const int tile = a.n_qtiles - 1 - tile_rev;  // the longest-running tiles launch first
  const int q_len = a.q_lens[r];
  const int q0 = tile * BQ;
  if (q0 >= q_len) return;
  const int ctx = a.ctx_lens[r];
  const int q_start = a.q_starts[r];
  const int kvh = blockIdx.y / a.hchunks;
  const int hc = blockIdx.y - kvh * a.hchunks;
  const int hg = wave % HG;
  const int qb = wave / HG;
  const int head = kvh * a.group + hc * HG + hg;
  const int past = ctx - q_len;  // position of query 0 is past + 0

  const int wq0 = q0 + qb * 32;
  const int qi = wq0 + col;
  const bool q_ok = qi < q_len;
  const int pos = past + qi;
  const int key_end = past + min(q0 + BQ, q_len);  // keys the workgroup needs
  const int wave_key_end = wq0 < q_len ? past + min(wq0 + 32, q_len) : 0;
  const int wave_pos_min = past + wq0;

  // Q^T as B operands: lane (col, half) holds d = 16 kc + 8 half .. + 7 of its query.
  V8 qreg[KC];
  {
    const T* qp = static_cast<const T*>(a.q) + static_cast<int64_t>(q_start + qi) * a.q_st +
                  static_cast<int64_t>(head) * a.q_sh + 8 * half;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      Pack16<T> x;
      if (q_ok) x = load16(qp + 16 * kc);
      else x.raw = u32x4{0, 0, 0, 0};
      qreg[kc] = __builtin_bit_cast(V8, x.raw);
    }
  }

  f32x16 oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) oacc[dt] = f32x16{};
  float m_run = -1.0e30f;  // running max of scale*log2e*score; finite, so 2^(m_run - x) is 0
  float l_run = 0.f;       // this lane half's share of the softmax denominator

  // Staging: thread tid copies unit `part` (8 elements) of keys KPT * kgrp .. + KPT - 1,
  // key groups fastest across lanes (so a transposed-V write spreads over the banks).
  const int kgrp = tid % NKG;
  const int part = tid / NKG;
  const int32_t* btrow = a.bt + static_cast<int64_t>(r) * a.bt_s;
  const T* kg = static_cast<const T*>(a.k) + static_cast<int64_t>(kvh) * a.k_sh + part * 8;
  const T* vg = static_cast<const T*>(a.v) + static_cast<int64_t>(kvh) * a.k_sh + part * 8;
  const int bs_mask = (1 << a.lbs) - 1;

  Pack16<T> kst[KPT], vst[KPT];
  int btv[KPT];  // block-table entries of the tile after the one being loaded
  auto fetch_bt = [&](int n0) {
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int n = n0 + kgrp * KPT + u;
      btv[u] = n < key_end ? btrow[n >> a.lbs] : 0;
    }
  };
  auto issue = [&](int n0) {
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int n = n0 + kgrp * KPT + u;
      if (n < key_end) {
        const int64_t off =
            ((static_cast<int64_t>(btv[u]) << a.lbs) + (n & bs_mask)) * a.k_ss;
        kst[u] = load16(kg + off);
        vst[u] = load16(vg + off);
      } else {
        kst[u].raw = u32x4{0, 0, 0, 0};  // keys past the tile's need: zeros, never NaN
        vst[u].raw = u32x4{0, 0, 0, 0};
      }
    }
  };

  fetch_bt(0);
  issue(0);
  if (kBN < key_end) fetch_bt(kBN);

  for (int n0 = 0; n0 < key_end; n0 += kBN) {
    __syncthreads();  // every wave is done reading the previous tile
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int key = kgrp * KPT + u;
      store16(k_lds + key * D + k_unit<CH>(key, part) * 8, kst[u]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = part * 8 + e;
      T* row = vt_lds + d * kBN;
      if constexpr (KPT == 4) {
        typedef T T4 __attribute__((ext_vector_type(4)));
        T4 x = {vst[0].v[e], vst[1].v[e], vst[2].v[e], vst[3].v[e]};
        *reinterpret_cast<T4*>(row + vt_col(kgrp * 4, d)) = x;
      } else {
        typedef T T2 __attribute__((ext_vector_type(2)));
        T2 x = {vst[0].v[e], vst[1].v[e]};
        *reinterpret_cast<T2*>(row + vt_col(kgrp * 2, d)) = x;
      }
    }
    __syncthreads();
    if (n0 + kBN < key_end) {
      issue(n0 + kBN);
      if (n0 + 2 * kBN < key_end) fetch_bt(n0 + 2 * kBN);
    }

    if (n0 >= wave_key_end) continue;  // this wave's queries are all before the tile

    // S^T = K . Q^T for the tile's two 32-key halves: two independent MFMA chains.
    f32x16 s0 = {}, s1 = {};
    {
      const T* kr0 = k_lds + col * D;
      const T* kr1 = kr0 + 32 * D;
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        const int u0 = k_unit<CH>(col, 2 * kc + half), u1 = k_unit<CH>(col + 32, 2 * kc + half);
        s0 = Mfma<T>::mma(*reinterpret_cast<const V8*>(kr0 + 8 * u0), qreg[kc], s0);
        s1 = Mfma<T>::mma(*reinterpret_cast<const V8*>(kr1 + 8 * u1), qreg[kc], s1);
      }
    }
    // Causal mask, only on a tile that crosses this wave's diagonal: item v of the lane
    // holds key n0 + 8 (v / 4) + 4 half + v % 4 (+ 32 in s1).
    if (n0 + kBN - 1 > wave_pos_min) {
      const int lim = pos - n0 - 4 * half;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int kofs = 8 * (v >> 2) + (v & 3);
        if (kofs > lim) s0[v] = -INFINITY;
        if (kofs + 32 > lim) s1[v] = -INFINITY;
      }
    }

    // Online softmax for this lane's query, in base 2 with the scale folded into one
    // FMA: p = 2^(s * c - m), c = scale * log2(e) > 0, so max(s) * c = max(s * c).
    float mx = fmaxf(s0[0], s1[0]);
#pragma unroll
    for (int v = 1; v < 16; ++v) mx = fmaxf(mx, fmaxf(s0[v], s1[v]));
    mx = halves_max(mx);
    const float m_new = fmaxf(m_run, mx * a.scale_log2);
    if (__any(m_new > m_run)) {  // rescale only when some lane's maximum moved
      const float alpha = fast_exp2(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
      m_run = m_new;
    }
    const float neg_m = -m_run;
    const float c = a.scale_log2;
    float psum = 0.f;
    V8 pk[4];
    V8 pk_lo[kSplitP ? 4 : 1];
    typedef float F2 __attribute__((ext_vector_type(2)));
    typedef T T2 __attribute__((ext_vector_type(2)));
    typedef T T4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int c0 = 0; c0 < 4; ++c0) {
      const f32x16& sv = (c0 < 2) ? s0 : s1;
      T2 h[4], lo[4];
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const int v = 8 * (c0 & 1) + 2 * e2;
        const F2 pf = {fast_exp2(fmaf(sv[v], c, neg_m)), fast_exp2(fmaf(sv[v + 1], c, neg_m))};
        psum += pf[0] + pf[1];
        h[e2] = __builtin_convertvector(pf, T2);
        if constexpr (kSplitP) lo[e2] = __builtin_convertvector(pf - __builtin_convertvector(h[e2], F2), T2);
      }
      const T4 a01 = __builtin_shufflevector(h[0], h[1], 0, 1, 2, 3);
      const T4 a23 = __builtin_shufflevector(h[2], h[3], 0, 1, 2, 3);
      pk[c0] = __builtin_shufflevector(a01, a23, 0, 1, 2, 3, 4, 5, 6, 7);
      if constexpr (kSplitP) {
        const T4 b01 = __builtin_shufflevector(lo[0], lo[1], 0, 1, 2, 3);
        const T4 b23 = __builtin_shufflevector(lo[2], lo[3], 0, 1, 2, 3);
        pk_lo[c0] = __builtin_shufflevector(b01, b23, 0, 1, 2, 3, 4, 5, 6, 7);
      }
    }
    l_run += psum;

    // O^T += V^T . P^T.
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int d = dt * 32 + col;
      const T* vr = vt_lds + d * kBN;
#pragma unroll
      for (int c0 = 0; c0 < 4; ++c0) {
        const V8 va = *reinterpret_cast<const V8*>(vr + (((2 * c0 + half) ^ vt_swz(d)) << 3));
        oacc[dt] = Mfma<T>::mma(va, pk[c0], oacc[dt]);
        if constexpr (kSplitP) oacc[dt] = Mfma<T>::mma(va, pk_lo[c0], oacc[dt]);
      }
    }
  }

  const float l_tot = halves_sum(l_run);
  if (!q_ok) return;
  T* op = static_cast<T*>(a.out) + static_cast<int64_t>(q_start + qi) * a.o_st +
          static_cast<int64_t>(head) * a.o_sh;
  const float inv = 1.f / l_tot;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      typedef T T4 __attribute__((ext_vector_type(4)));
      T4 x;
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = static_cast<T>(oacc[dt][4 * j + i] * inv);
      *reinterpret_cast<T4*>(op + dt * 32 + 8 * j + 4 * half) = x;
    }
}

template <typename T, int D, int HG>
static int launch_prefill_mfma(const PrefillArgs& a, int Hkv, hipStream_t stream) {
  constexpr int QB = 4 / HG;
  dim3 grid(static_cast<unsigned>(a.n_qtiles) * a.R, Hkv * a.hchunks);
  hipLaunchKernelGGL((prefill_mfma_kernel<T, D, HG, QB>), grid, dim3(kThreads), 0, stream, a);
  return launch_status();
}

template <typename T, int D>
static int dispatch_hg(PrefillArgs& a, int Hkv, int max_q_len, hipStream_t stream) {
  const int hg = a.group < 4 ? a.group : 4;
  a.hchunks = a.group / hg;
  const int bq = 32 * (4 / hg);
  a.n_qtiles = (max_q_len + bq - 1) / bq;
  switch (hg) {
    case 1: return launch_prefill_mfma<T, D, 1>(a, Hkv, stream);
    case 2: return launch_prefill_mfma<T, D, 2>(a, Hkv, stream);
    case 4: return launch_prefill_mfma<T, D, 4>(a, Hkv, stream);
    default: return TS_EUNSUPPORTED;
  }
}

int prefill_rows_generic(const void* q, const void* k, const void* v, void* out,
                         const int32_t* bt, const int32_t* q_starts, const int32_t* q_lens,
                         const int32_t* ctx_lens, int R, int Hq, int Hkv, int D, int lbs,
                         int max_q_len, int64_t q_st, int64_t q_sh, int64_t o_st, int64_t o_sh,
                         int64_t k_ss, int64_t k_sh, int64_t bt_s, float scale, int dtype,
                         hipStream_t stream);

}  // namespace ts

using namespace ts;

extern "C" int ts_prefill_varlen(const void* q, const void* k_cache, const void* v_cache,
                                 void* out, const int32_t* block_tables,
                                 const int32_t* q_starts, const int32_t* q_lens,
                                 const int32_t* context_lens, int R, int Hq, int Hkv, int D,
                                 int block_size, int max_q_len, int64_t q_stride_t,
                                 int64_t q_stride_h, int64_t o_stride_t, int64_t o_stride_h,
                                 int64_t k_stride_slot, int64_t k_stride_head,
                                 int64_t bt_stride, float scale, int dtype, void* stream) {
  if (R < 0 || max_q_len < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || !is_pow2(Hq / Hkv) ||
      !is_pow2(block_size))
    return TS_EINVAL;
  if (R == 0 || max_q_len == 0) return 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int lbs = ilog2(block_size);
  if ((dtype == TS_F16 || dtype == TS_BF16) && (D == 64 || D == 128)) {
    PrefillArgs a{q, k_cache, v_cache, out, block_tables, q_starts, q_lens, context_lens,
                  R, Hq / Hkv, 1, lbs, 1, q_stride_t, q_stride_h, o_stride_t, o_stride_h,
                  k_stride_slot, k_stride_head, bt_stride, scale * kLog2e};
    if (dtype == TS_F16) {
      return D == 64 ? dispatch_hg<f16, 64>(a, Hkv, max_q_len, st)
                     : dispatch_hg<f16, 128>(a, Hkv, max_q_len, st);
    }
    return D == 64 ? dispatch_hg<bf16, 64>(a, Hkv, max_q_len, st)
                   : dispatch_hg<bf16, 128>(a, Hkv, max_q_len, st);
  }
  return prefill_rows_generic(q, k_cache, v_cache, out, block_tables, q_starts, q_lens,
                              context_lens, R, Hq, Hkv, D, lbs, max_q_len, q_stride_t,
                              q_stride_h, o_stride_t, o_stride_h, k_stride_slot,
                              k_stride_head, bt_stride, scale, dtype, st);
}
