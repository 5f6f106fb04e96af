// Paged GQA decode attention for gfx950: one wave64 per (sequence, query-head tile,
// split), the split-K combine pass, and the same loop reused as the generic (fp32 /
// small head_dim) varlen prefill path.
//
// Reference behaviour: src/tinyserve/triton_attention.py:76-327 (per-head, grouped and
// split kernels, merge kernel), numerics of src/tinyserve/attention.py:62-141.
//
// Lane layout. A head row of D elements is read by LPT consecutive lanes ("lanes per
// token"), each holding E = D / LPT elements as 16-byte vectors; vector i of lane c
// covers elements (i * LPT + c) * VEC .. + VEC - 1, so one load instruction of the LPT
// lanes of a token reads LPT * 16 contiguous bytes. A wave therefore streams
// TPW = 64 / LPT tokens per iteration (16 tokens of a 16-slot block for fp16 D=128:
// 4 KB of K and 4 KB of V per wave per iteration, issued before the previous
// iteration's math so that two or three iterations are in flight, by register budget).
//
// Waves per workgroup. A decode launch gives each (sequence, head tile, split) a
// workgroup of W = 1, 2, 4 (or, under the light budget below, 8) waves; wave w takes the
// w-th of W contiguous block ranges of the split's range, and the W partial states are
// merged through LDS before anything is written. This is split-K without HBM partials or a second launch: the library picks W
// so that the grid holds about four waves per CU (the kernel's heavy register budget
// needs more than 256 VGPRs, so a SIMD runs one wave of it, and a CU wants four in
// flight to cover HBM latency). Launches of two or more rounds of such waves (many
// sequences, or many splits) take the light budget instead: 32 bytes per lane, two waves
// per SIMD, so that one wave's start-up chain and merge hide under another's streaming.
//
// Length pairs. A batch of at most 64 sequences that would get two-wave workgroups is
// run as pairs instead: workgroup y takes the sequences ranked y and B - 1 - y by
// length (longest with shortest), and its four waves take equal shares of the two
// sequences' blocks laid end to end (one wave may walk the end of one and the start of
// the other). Every workgroup then has about the same work, so a batch of mixed
// lengths does not wait on its longest sequences; equal lengths give the two-wave
// layout again.
//
// Softmax. Every token lane keeps its own running (max, sum, acc) per query head (the
// online softmax of triton_attention.py:14-22, in base 2), so the loop has no
// cross-lane work except the LPT-lane dot-product reduction. The token lanes are
// merged once at the end with the two-partial rule m = max(m1, m2),
// l = 2^(m1-m) l1 + 2^(m2-m) l2 (same for acc), the rule the combine pass uses too.
#include <algorithm>
#include <mutex>

#include "common.h"

namespace ts {

// Two register budgets. kHeavy: each lane streams 64 bytes of a head row per token, three
// iterations in flight, one wave per SIMD (more than 256 VGPRs) -- for launches whose
// waves all run in one round, where each wave must keep much in flight. kLight: 32 bytes
// per lane, two in flight, two waves per SIMD -- for launches of several rounds, where
// the second wave per SIMD hides each wave's start-up chain (lengths, block table, first
// loads) and merge. (Tiles of four query heads stream 16 bytes per lane under it, or
// their state would spill.) kLightStream is kLight with K/V read by non-temporal loads,
// for decode launches larger than the last-level cache.
enum Budget { kHeavy = 0, kLight = 1, kLightStream = 2 };
template <int B>
struct BudgetOf {
  static constexpr bool kLightish = B != kHeavy;
  static constexpr int kLaneBytes = kLightish ? 32 : 64;
  // Iterations in flight. Two under the light budgets: with two waves per SIMD a third
  // only adds loads in flight past what HBM serves best (measured +0.3% to +2.5%
  // with two, headline included).
  static constexpr int kNBuf = kLightish ? 2 : 3;
  static constexpr int kWavesPerEU = kLightish ? 2 : 1;
};

template <typename T, int D, int LB>
struct RowShape {
  static constexpr int kRowBytes = D * static_cast<int>(sizeof(T));
  static constexpr int kLaneBytes = LB;  // bytes of a row per lane
  static constexpr int kLPT =
      kRowBytes <= kLaneBytes ? 1 : (kRowBytes / kLaneBytes > 64 ? 64 : kRowBytes / kLaneBytes);
  static constexpr int kE = D / kLPT;
  static constexpr int kVec = 16 / static_cast<int>(sizeof(T));
  static constexpr int kNV = kE / kVec;
  static constexpr int kTPW = kWave / kLPT;
  static_assert(kNV >= 1 && kNV * kVec == kE, "a head row must be a multiple of 16 bytes");
};

struct AttendArgs {
  const void* q;
  const void* k;
  const void* v;
  const int32_t* bt;
  const int32_t* lens;  // decode: context_lens; prefill: context_lens of each sequence
  void* out;
  float* m;
  float* l;
  float* acc;
  const int32_t* q_starts;  // prefill only
  const int32_t* q_lens;    // prefill only
  int Hq;
  int group;  // query heads per kv head
  int lbs;    // log2(block_size)
  int splits;
  int wpg;        // waves per workgroup (decode), 1 for prefill
  int max_q_len;  // prefill only
  int by_length;  // decode: workgroup y takes the sequences of length rank y and nseq-1-y
  int nseq;       // decode: sequences in the batch
  int64_t q_sb, q_sh, o_sb, o_sh, k_ss, k_sh, bt_s;
  float scale_log2;  // softmax scale * log2(e)
  int stream_kv;     // decode, light budget: K/V through non-temporal loads
  // decode, in-workgroup split-K: the walk of each sequence is cut at the block ranges of
  // `cuts` splits (split s: blocks [s * ceil(n / cuts), ...), the reference's ranges);
  // every range piece's softmax state is parked in LDS and the workgroup merges them. 0:
  // no cuts (the workgroup's waves merge one state each).
  int cuts;
  int width;  // decode: block-table width when at most 64 (the row is loaded up front), else 0
};

// Partial dot product of one 16-byte K vector with the matching q vector, fp32 result
// (v_dot2_f32_{f16,bf16}: two products per instruction, fp32 accumulation).
__device__ __forceinline__ float dot16(const Pack16<f16>& a, const Pack16<f16>& b, float s) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const h2 x = {a.v[2 * j], a.v[2 * j + 1]};
    const h2 y = {b.v[2 * j], b.v[2 * j + 1]};
    s = __builtin_amdgcn_fdot2(x, y, s, false);
  }
  return s;
}
__device__ __forceinline__ float dot16(const Pack16<bf16>& a, const Pack16<bf16>& b, float s) {
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const b2 x = {a.v[2 * j], a.v[2 * j + 1]};
    const b2 y = {b.v[2 * j], b.v[2 * j + 1]};
    s = __builtin_amdgcn_fdot2_f32_bf16(x, y, s, false);
  }
  return s;
}
__device__ __forceinline__ float dot16(const Pack16<float>& a, const Pack16<float>& b, float s) {
#pragma unroll
  for (int j = 0; j < 4; ++j) s = fmaf(a.v[j], b.v[j], s);
  return s;
}

template <typename T, int D, int HT, int LB>
struct TokenState {
  using S = RowShape<T, D, LB>;
  float m[HT];
  float l[HT];
  float acc[HT][S::kE];
};

// Max over lanes OFF, 2 OFF, ... apart.
template <int OFF>
__device__ __forceinline__ float token_lanes_max(float x) {
  if constexpr (OFF < 64) return token_lanes_max<OFF * 2>(fmaxf(x, xor_lane<OFF>(x)));
  return x;
}
// Sum over lanes OFF, 2 OFF, ... apart. DPP: the exchange folds into the add (row
// rotations within 16 lanes, then v_permlane16_swap / v_permlane32_swap), the shorter
// dependency chain for launches bound by latency; otherwise ds_swizzle / ds_bpermute,
// which run beside the VALU for launches bound by issue.
template <int OFF, bool DPP>
__device__ __forceinline__ float token_lanes_sum(float x) {
  if constexpr (OFF >= 64) {
    return x;
  } else if constexpr (!DPP) {
    return token_lanes_sum<OFF * 2, DPP>(x + xor_lane<OFF>(x));
  } else if constexpr (OFF < 16) {
    // Rotating each 16-lane row by OFF, 2 OFF, ..., 8 and adding sums the lanes of the
    // row that agree mod OFF.
    const float y = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x120 + OFF, 0xf, 0xf, false));
    return token_lanes_sum<OFF * 2, DPP>(x + y);
  } else if constexpr (OFF == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return token_lanes_sum<32, DPP>(__uint_as_float(r[0]) + __uint_as_float(r[1]));
  } else {
    return halves_sum(x);
  }
}

// Merge the states of a wave's token lanes (lanes LPT, 2 LPT, ... apart) into one held
// by every lane: the common maximum first, then each lane rescales its own state once
// and the rescaled states are summed (one exponential per head instead of two per
// exchange level).
template <bool DPP, typename T, int D, int HT, int LB>
__device__ __forceinline__ void merge_token_lanes(TokenState<T, D, HT, LB>& st) {
  constexpr int L = RowShape<T, D, LB>::kLPT;
  using S = RowShape<T, D, LB>;
  if constexpr (L < 64) {
#pragma unroll
    for (int g = 0; g < HT; ++g) {
      const float mn = token_lanes_max<L>(st.m[g]);
      const float f = fast_exp2(st.m[g] - mn);
      st.l[g] = token_lanes_sum<L, DPP>(st.l[g] * f);
#pragma unroll
      for (int e = 0; e < S::kE; ++e) st.acc[g][e] = token_lanes_sum<L, DPP>(st.acc[g][e] * f);
      st.m[g] = mn;
    }
  }
}

constexpr int kMaxWavesPerGroup = 4;  // heavy budget, and length pairs
constexpr int kMaxWavesLight = 8;     // light budget (two waves per SIMD)

// LDS of a decode workgroup (dynamic, sized by the launch): NS state slots, each the
// HT maxima, HT denominators and HT x D accumulators of one wave's merged state. A plain
// workgroup of W > 1 waves parks one state per wave (NS = W); a length pair parks up to
// two per wave, one per sequence it walked (NS = 2W, slot 2w + i). One-wave workgroups
// take none.
template <int HT, int D>
struct StateSlots {
  float* base;
  int ns;
  __device__ float& m(int s, int g) const { return base[s * HT + g]; }
  __device__ float& l(int s, int g) const { return base[(ns + s) * HT + g]; }
  __device__ float& acc(int s, int g, int d) const { return base[2 * ns * HT + (s * HT + g) * D + d]; }
};

__host__ __device__ constexpr int64_t state_slot_bytes(int ht, int d) {
  return static_cast<int64_t>(ht) * (d + 2) * 4;
}

// Lanes c (c >= 0: the first LPT lanes of a wave, lane c holding elements
// (i * LPT + c) * VEC + j) write their merged state to slot s.
template <typename State, typename Slots>
__device__ __forceinline__ void park_state(const Slots& ss, const State& st, int s, int c) {
  using S = typename State::S;
  constexpr int NV = S::kNV, VEC = S::kVec, LPT = S::kLPT;
  constexpr int HT = sizeof(st.m) / sizeof(float);
  if (c < 0) return;
#pragma unroll
  for (int g = 0; g < HT; ++g) {
    if (c == 0) {
      ss.m(s, g) = st.m[g];
      ss.l(s, g) = st.l[g];
    }
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
      for (int j = 0; j < VEC; ++j) ss.acc(s, g, (i * LPT + c) * VEC + j) = st.acc[g][i * VEC + j];
  }
}

// Sum over lanes OFF, 2 OFF, ..., 8 apart (within each 16-lane row).
template <int OFF, bool DPP>
__device__ __forceinline__ float row_lanes_sum(float x) {
  if constexpr (OFF >= 16) {
    return x;
  } else if constexpr (DPP) {
    const float y = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x120 + OFF, 0xf, 0xf, false));
    return row_lanes_sum<OFF * 2, DPP>(x + y);
  } else {
    return row_lanes_sum<OFF * 2, DPP>(x + xor_lane<OFF>(x));
  }
}

// Merge the token lanes' states and park the result in slot s. Common maximum and one
// rescale per lane as in merge_token_lanes, then a reduce-scatter of the accumulators
// over the token lanes 32 and 16 apart: v_permlane32_swap (v_permlane16_swap) of the
// register pair (upper half, lower half) of the elements hands each lane its partner's
// copy of the half it keeps (lanes 0-31, even rows: the upper half), so each level is
// one swap and one add per pair, and halves what a lane holds. Token lanes closer than
// 16 are summed whole. Each lane then writes its E / 4 (E / 2) elements.
template <bool DPP, typename T, int D, int HT, int LB>
__device__ __forceinline__ void merge_park(const StateSlots<HT, D>& ss, TokenState<T, D, HT, LB>& st,
                                           int s) {
  using S = RowShape<T, D, LB>;
  constexpr int L = S::kLPT, E = S::kE, VEC = S::kVec;
  const int lane = threadIdx.x % kWave;
  if constexpr (L >= 64) {
    park_state(ss, st, s, lane);
  } else {
    constexpr bool H32 = L <= 32, H16 = L <= 16;
    constexpr int Q = E >> ((H32 ? 1 : 0) + (H16 ? 1 : 0));
    int o = 0;
    if constexpr (H32) o += lane < 32 ? E / 2 : 0;
    if constexpr (H16) o += ((lane >> 4) & 1) == 0 ? E / 4 : 0;
    const int c = lane % L;
    const bool writer = L >= 16 || (lane & 15) < L;
#pragma unroll
    for (int g = 0; g < HT; ++g) {
      const float mn = token_lanes_max<L>(st.m[g]);
      const float f = fast_exp2(st.m[g] - mn);
      const float l = token_lanes_sum<L, DPP>(st.l[g] * f);
      float x[E];
#pragma unroll
      for (int e = 0; e < E; ++e) x[e] = st.acc[g][e] * f;
      if constexpr (H32) {
#pragma unroll
        for (int i = 0; i < E / 2; ++i) {
          const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x[E / 2 + i]), __float_as_uint(x[i]), false, false);
          x[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        }
      }
      if constexpr (H16) {
#pragma unroll
        for (int i = 0; i < E / 4; ++i) {
          const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x[E / 4 + i]), __float_as_uint(x[i]), false, false);
          x[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        }
      }
#pragma unroll
      for (int q = 0; q < Q; ++q) x[q] = row_lanes_sum<L, DPP>(x[q]);
      if (lane == 0) {
        ss.m(s, g) = mn;
        ss.l(s, g) = l;
      }
      if (writer) {
#pragma unroll
        for (int q = 0; q < Q; ++q) {
          const int e = o + q;
          ss.acc(s, g, ((e / VEC) * L + c) * VEC + e % VEC) = x[q];
        }
      }
    }
  }
}

// The W waves of a decode workgroup have each parked a merged state in slot w; then
// thread t of the group produces output element t (of HT * D) by the two-partial rule
// over the W states, and writes it either as the final output (one split) or as the
// split's fp32 partial for the combine pass.
template <typename T, int D, int HT, typename Args>
__device__ __forceinline__ void merge_group_waves(const Args& a, const StateSlots<HT, D>& ss,
                                                  int seq, int h0, int split, int64_t orow) {
  __syncthreads();
  const int W = a.wpg;
  for (int t = threadIdx.x; t < HT * D; t += W * kWave) {
    const int g = t / D, d = t % D;
    float mm = ss.m(0, g);
    for (int w = 1; w < W; ++w) mm = fmaxf(mm, ss.m(w, g));
    float den = 0.f, num = 0.f;
    for (int w = 0; w < W; ++w) {
      const float f = fast_exp2(ss.m(w, g) - mm);
      den = fmaf(f, ss.l(w, g), den);
      num = fmaf(f, ss.acc(w, g, d), num);
    }
    if (a.splits == 1) {
      static_cast<T*>(a.out)[orow + (h0 + g) * a.o_sh + d] = from_f32<T>(num / den);
    } else {
      const int64_t part = (static_cast<int64_t>(seq) * a.Hq + h0 + g) * a.splits + split;
      if (d == 0) {
        a.m[part] = den > 0.f ? mm : -INFINITY;
        a.l[part] = den;
      }
      a.acc[part * D + d] = num;
    }
  }
}

// A finite "no score yet" maximum: 2^(kNoMax - real score) is exactly 0, and two empty
// states merge to an empty state without inf - inf.
constexpr float kNoMax = -1.0e30f;

template <typename T, int D, int HT, bool PREFILL, int BUDGET, bool CUT = false>
__global__ __launch_bounds__(PREFILL ? kWave : kWave * (BudgetOf<BUDGET>::kLightish ? kMaxWavesLight : kMaxWavesPerGroup))
__attribute__((amdgpu_waves_per_eu(BudgetOf<BUDGET>::kWavesPerEU)))
void paged_attend_kernel(const AttendArgs a) {
  // Under the light budget four query heads' state fits only at 16 bytes per lane.
  constexpr int LB = BudgetOf<BUDGET>::kLightish && HT == 4 ? 16 : BudgetOf<BUDGET>::kLaneBytes;
  using S = RowShape<T, D, LB>;
  constexpr int LPT = S::kLPT, NV = S::kNV, VEC = S::kVec, TPW = S::kTPW, E = S::kE;
  // Streaming launches are bound by issue, cached ones (short walks) by latency.
  constexpr bool kDppMerge = BUDGET != kLightStream;
  constexpr int NBUF = BudgetOf<BUDGET>::kNBuf;
  const int lane = threadIdx.x % kWave;
  const int wave = PREFILL ? 0 : threadIdx.x / kWave;
  const int c = lane % LPT;
  const int tl = lane / LPT;
  // Decode grid (head tiles, sequences, splits): the head tiles of one sequence are
  // dispatched together, so the kv heads of a slot (one contiguous 2 KB row at Qwen3
  // shapes) are read at about the same time. Prefill grid (rows, head tiles).
  const int h0 = (PREFILL ? blockIdx.y : blockIdx.x) * HT;
  const int kvh = h0 / a.group;

  int seq, ctx, split = 0;
  int64_t qrow, orow;
  // Length pairs: the two sequences, and this wave's segments (sequence, block range).
  int pair_a = -1, pair_b = -1, len_a = 0, len_b = 0, n_a = 0, share = 1, nseg = 1;
  int seg_seq[2] = {0, 0}, seg_first[2] = {0, 0}, seg_last[2] = {0, 0};
  // Decode, a narrow table (at most 64 blocks) and no pairs: the sequence's whole row is
  // loaded first, one entry per lane, in parallel with its context length instead of
  // after it.
  int win_pre = 0;
  if constexpr (PREFILL) {
    seq = blockIdx.x / a.max_q_len;
    const int i = blockIdx.x - seq * a.max_q_len;
    const int ql = a.q_lens[seq];
    if (i >= ql) return;  // the grid covers the longest sequence
    const int row = a.q_starts[seq] + i;
    ctx = a.lens[seq] - ql + i + 1;  // causal: keys 0 .. its own position
    qrow = row * a.q_sb;
    orow = row * a.o_sb;
  } else {
    seq = blockIdx.y;
    if (!a.by_length && a.width > 0) win_pre = lane < a.width ? a.bt[seq * a.bt_s + lane] : 0;
    if (a.by_length) {
      // Workgroup y takes the sequences ranked y and B - 1 - y by length (longest
      // first, ties by index): lane b ranks sequence b against the others (B <= 64).
      // Its waves are shared between the two in proportion to their lengths, so every
      // workgroup has about the same work and all run in one round.
      const int B = a.nseq;
      const int mine = lane < B ? a.lens[lane] : -1;
      // A batch already in that order (equal lengths included) needs no ranking.
      const int next = __shfl_down(mine, 1);
      int rank = lane;
      if (!__all(lane + 1 >= B || mine >= next)) {
        rank = 0;
        if (__all(mine < (1 << 25))) {
          // Unique keys (length, then lower index first): rank = keys above this one.
          const int key = lane < B ? mine * kWave + (kWave - 1 - lane) : -1;
          for (int j = 0; j < B; ++j) rank += __builtin_amdgcn_readlane(key, j) > key;
        } else {
          for (int j = 0; j < B; ++j) {
            const int other = __builtin_amdgcn_readlane(mine, j);
            rank += (other > mine) | ((other == mine) & (j < lane));
          }
        }
      }
      const int ra = blockIdx.y, rb = B - 1 - ra;
      pair_a = __builtin_ctzll(__ballot(lane < B && rank == ra));
      pair_b = rb != ra ? __builtin_ctzll(__ballot(lane < B && rank == rb)) : -1;
      len_a = __builtin_amdgcn_readlane(mine, pair_a);
      len_b = pair_b >= 0 ? __builtin_amdgcn_readlane(mine, pair_b) : 0;
      // The waves take equal shares of the two sequences' blocks laid end to end; at
      // most one wave's share straddles both, and it walks them one after the other.
      const int bmask = (1 << a.lbs) - 1;
      n_a = (len_a + bmask) >> a.lbs;
      const int n_b = (len_b + bmask) >> a.lbs;
      share = (n_a + n_b + a.wpg - 1) / a.wpg;
      const int lo = min(wave * share, n_a + n_b), hi = min(lo + share, n_a + n_b);
      nseg = 0;
      if (lo < n_a) {
        seg_seq[nseg] = pair_a, seg_first[nseg] = lo, seg_last[nseg] = min(hi, n_a);
        ++nseg;
      }
      if (hi > n_a) {
        seg_seq[nseg] = pair_b, seg_first[nseg] = max(lo, n_a) - n_a, seg_last[nseg] = hi - n_a;
        ++nseg;
      }
      seq = pair_a;
    }
    split = blockIdx.z;
    ctx = a.by_length ? len_a : a.lens[seq];
    qrow = seq * a.q_sb;
    orow = seq * a.o_sb;
  }
  const int lbs = a.lbs;
  const int bs_mask = (1 << lbs) - 1;
  const int nblocks = (ctx + bs_mask) >> lbs;
  // Split s covers blocks [s * ceil(n / S), ...) of the sequence, clipped to n (the
  // reference's ranges, triton_attention.py:283-286, so each partial holds the same
  // keys); the W waves of its workgroup take equal contiguous shares of that range.
  const int per_split = (nblocks + a.splits - 1) / a.splits;
  const int s_first = min(split * per_split, nblocks);
  const int s_last = min(s_first + per_split, nblocks);
  const int nw = PREFILL ? 1 : a.wpg;
  const int per = (s_last - s_first + nw - 1) / nw;
  int first = s_first + wave * per;
  int last = min(first + per, s_last);
  bool pair = false;
  if constexpr (!PREFILL) pair = a.by_length;
  if (!pair) seg_seq[0] = seq, seg_first[0] = first, seg_last[0] = last;

  // Cut mode: a wave's walk of one sequence is cut at every multiple of that sequence's
  // split length pc = ceil(n / cuts) blocks into pieces, each with its own softmax state
  // parked in LDS. The piece of split k walked by wave w takes slot k + w (+ cuts + W for
  // the second sequence of a length pair): along a sequence's blocks both k and w only
  // grow, and at least one of them grows from one piece to the next, so slots never
  // collide. Slots no piece takes are marked before the walk (m = -1e30) and skipped; the
  // merge takes the other slots of a sequence in slot order (position order, so the
  // result does not depend on timing).
  TokenState<T, D, HT, LB> st;
  extern __shared__ float lds_slots[];
  const StateSlots<HT, D> ss{lds_slots, CUT ? (pair ? 2 : 1) * (a.cuts + nw)
                                            : (pair ? 2 : 1) * (PREFILL ? 1 : a.wpg)};
  if constexpr (CUT) {
    // An unused slot is marked by its maximum alone; the merge skips it.
    for (int i = threadIdx.x; i < ss.ns * HT; i += nw * kWave) lds_slots[i] = kNoMax;
    __syncthreads();
  }
  for (int sgi = 0; sgi < nseg; ++sgi) {
  if (pair) {
    seq = seg_seq[sgi];
    ctx = seq == pair_a ? len_a : len_b;
    qrow = seq * a.q_sb;
    first = seg_first[sgi];
    last = seg_last[sgi];
  }
  // Cut mode: this segment's first slot, and the next split boundary (tokens); set once
  // the segment's first loads are in flight.
  const int cut_seq = pair && seq != pair_a ? 1 : 0;
  int slot = 0, next_cut = 0x7fffffff, pc_tokens = 0;
  auto cut_setup = [&]() {
    const int n = (ctx + bs_mask) >> lbs;
    const int pc = __builtin_amdgcn_readfirstlane(max(1, (n + a.cuts - 1) / a.cuts));
    const int k = __builtin_amdgcn_readfirstlane(first / pc);
    slot = cut_seq * (a.cuts + nw) + k + wave;
    pc_tokens = pc << lbs;
    next_cut = (k + 1) * pc_tokens;
  };
  const T* qp = static_cast<const T*>(a.q) + qrow;
  Pack16<T> qv[HT][NV];
#pragma unroll
  for (int g = 0; g < HT; ++g)
#pragma unroll
    for (int i = 0; i < NV; ++i) qv[g][i] = load16(qp + (h0 + g) * a.q_sh + (i * LPT + c) * VEC);

#pragma unroll
  for (int g = 0; g < HT; ++g) {
    st.m[g] = kNoMax;
    st.l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) st.acc[g][e] = 0.f;
  }

  if (first < last) {
    const int t0 = first << lbs;
    const int t1 = min(last << lbs, ctx);
    const int32_t* btrow = a.bt + seq * a.bt_s;
    const T* kbase = static_cast<const T*>(a.k) + kvh * a.k_sh + c * VEC;
    const T* vbase = static_cast<const T*>(a.v) + kvh * a.k_sh + c * VEC;
    // Lane j holds block-table entry `chunk + j`: a window of 64 blocks, refreshed when
    // the positions pass its end. An iteration never straddles two windows (it covers
    // TPW <= 64 positions starting at a multiple of TPW from a window start).
    int chunk = first;
    int win;
    if (!pair && a.width > 0) {
      chunk = 0;  // the whole row (at most 64 blocks) is in win_pre
      win = win_pre;
    } else {
      win = (chunk + lane < last) ? btrow[chunk + lane] : 0;
    }

    // NBUF iterations in flight: the loads of iteration i + NBUF - 1 are issued before
    // iteration i's math (ring of NBUF register buffers, indices fixed by unrolling).
    Pack16<T> kb[NBUF][NV], vb[NBUF][NV];
    // A wave's own query row, already read: the target of issues past the range.
    const T* const qdummy = qp + h0 * a.q_sh + c * VEC;
    auto issue = [&](Pack16<T>(&kf)[NV], Pack16<T>(&vf)[NV], int p0, bool live) {
      if (((p0 >> lbs) - chunk) >= 64) {
        chunk += 64;
        win = (chunk + lane < last) ? btrow[chunk + lane] : 0;
      }
      const int pos = p0 + tl;
      // A lane past the range reads the range's first token (owned and finite) and
      // is masked out of the softmax below.
      const int pe = pos < t1 ? pos : p0;
      const int blk = __shfl(win, (pe >> lbs) - chunk);
      const int64_t off = ((static_cast<int64_t>(blk) << lbs) + (pe & bs_mask)) * a.k_ss;
      const T* const kp = live ? kbase + off : qdummy;
      const T* const vp = live ? vbase + off : qdummy;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        if constexpr (BUDGET == kLightStream) {
          kf[i].raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kp + i * LPT * VEC));
          vf[i].raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vp + i * LPT * VEC));
        } else {
          kf[i] = load16(kp + i * LPT * VEC);
          vf[i] = load16(vp + i * LPT * VEC);
        }
      }
    };
    auto attend = [&](const Pack16<T>(&kf)[NV], const Pack16<T>(&vf)[NV], int p0) {
      const bool valid = p0 + tl < t1;
      float s[HT];
      bool grow = false;
#pragma unroll
      for (int g = 0; g < HT; ++g) {
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i) d = dot16(kf[i], qv[g][i], d);
        d = group_sum<LPT>(d) * a.scale_log2;
        s[g] = valid ? d : -INFINITY;
        grow |= s[g] > st.m[g];
      }
      float vf32[E];
#pragma unroll
      for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int j = 0; j < VEC; ++j) vf32[i * VEC + j] = to_f32(vf[i].v[j]);
      // The branch only rescales, in place; the update is common to both paths, so the
      // state keeps its registers (two paths that each wrote a new state made the
      // compiler copy it at their join).
      if (__any(grow)) {
#pragma unroll
        for (int g = 0; g < HT; ++g) {
          const float mn = fmaxf(st.m[g], s[g]);
          const float al = fast_exp2(st.m[g] - mn);
          st.l[g] *= al;
#pragma unroll
          for (int e = 0; e < E; ++e) st.acc[g][e] *= al;
          st.m[g] = mn;
        }
      }
#pragma unroll
      for (int g = 0; g < HT; ++g) {
        const float p = fast_exp2(s[g] - st.m[g]);
        st.l[g] += p;
#pragma unroll
        for (int e = 0; e < E; ++e) st.acc[g][e] = fmaf(p, vf32[e], st.acc[g][e]);
      }
    };

#pragma unroll
    // Every issue is unconditional: one past the range reads the wave's query row
    // instead (cached; its table lookup uses a position in range). A conditional issue
    // makes the compiler's load counting allow for the path where nothing was issued, and
    // each iteration's wait for its own data then also waits for the loads just issued.
    for (int j = 0; j + 1 < NBUF; ++j)
      issue(kb[j], vb[j], t0 + j * TPW < t1 ? t0 + j * TPW : t0, t0 + j * TPW < t1);
    if constexpr (CUT) cut_setup();
    for (int base = t0; base < t1; base += NBUF * TPW) {
#pragma unroll
      for (int j = 0; j < NBUF; ++j) {
        const int p0 = base + j * TPW;
        if (p0 >= t1) break;
        const int pn = p0 + (NBUF - 1) * TPW;
        issue(kb[(j + NBUF - 1) % NBUF], vb[(j + NBUF - 1) % NBUF], pn < t1 ? pn : p0, pn < t1);
        attend(kb[j], vb[j], p0);
        if constexpr (CUT) {
          // A split boundary (a whole number of iterations past t0: the host runs cut
          // mode only when TPW divides the block size): park this piece, start the next.
          if (p0 + TPW == next_cut && next_cut < t1) {
            merge_park<kDppMerge>(ss, st, slot++);
            // Only the maximum is reset: a lane's first token of the next piece raises
            // it and rescales the old l and acc by 2^(kNoMax - m) = 0, and a lane that
            // sees no token of the piece keeps m = kNoMax, which the merge weighs by 0
            // (every piece has a token, so the merged maximum is finite). Zeroing l and
            // acc here made the compiler copy the whole state through every iteration.
#pragma unroll
            for (int g = 0; g < HT; ++g) st.m[g] = kNoMax;
            next_cut += pc_tokens;
          }
        }
      }
    }
  }

  // Parked states are merged across waves below; a one-wave workgroup writes its own.
  if constexpr (CUT) {
    if (first < last) merge_park<kDppMerge>(ss, st, slot);
  } else if (pair) {
    merge_park<kDppMerge>(ss, st, 2 * wave + sgi);
  } else if (!PREFILL && a.wpg > 1) {
    merge_park<kDppMerge>(ss, st, wave);
  } else {
    merge_token_lanes<kDppMerge>(st);
  }
  }  // segments
  if constexpr (CUT) {
    // Every piece of a sequence, in position order, by the two-partial rule: the
    // sequence's result is the merge of its split ranges' states (each range possibly in
    // several pieces, merged by the same rule).
    __syncthreads();
    const int parts = pair && pair_b >= 0 ? 2 : 1;
    const int nsl = a.cuts + nw;  // slots per sequence (at most 16 + 8)
    for (int t = threadIdx.x; t < parts * HT * D; t += nw * kWave) {
      const int pi = t / (HT * D);
      const int g = (t % (HT * D)) / D, d = t % D;
      const int s0 = pi * nsl;
      float den = 0.f, num = 0.f;
      if (D % kWave == 0 && nsl <= kWave) {
        // A wave's 64 outputs share (sequence, head): lane s takes slot s's maximum and
        // denominator, the wave forms every slot's weight at once (one exponential per
        // lane), and the weights are broadcast slot by slot for the accumulators. (More
        // than 64 slots, possible at small states, take the loop below.)
        // An unused slot has only its maximum written: its other fields are never read.
        const float ms = lane < nsl ? ss.m(s0 + lane, g) : kNoMax;
        const float ls = ms != kNoMax ? ss.l(s0 + lane, g) : 0.f;
        float mm = ms;
        mm = fmaxf(mm, xor_lane<1>(mm));
        mm = fmaxf(mm, xor_lane<2>(mm));
        mm = fmaxf(mm, xor_lane<4>(mm));
        mm = fmaxf(mm, xor_lane<8>(mm));
        mm = fmaxf(mm, xor_lane<16>(mm));
        mm = halves_max(mm);
        // No piece: the slot's maximum is kNoMax, its weight 0 (a piece has a token, so
        // a finite maximum).
        const float f = ms == kNoMax ? 0.f : fast_exp2(ms - mm);
        den = group_sum<64>(ms != kNoMax ? f * ls : 0.f);
        for (int s2 = 0; s2 < nsl; ++s2) {
          const float fs = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), s2));
          if (fs != 0.f) num = fmaf(fs, ss.acc(s0 + s2, g, d), num);
        }
      } else {
        const int s1 = s0 + nsl;
        float mm = kNoMax;
        for (int s2 = s0; s2 < s1; ++s2) mm = fmaxf(mm, ss.m(s2, g));
        for (int s2 = s0; s2 < s1; ++s2) {
          const float ms = ss.m(s2, g);
          if (ms == kNoMax) continue;  // no piece (a piece has a token, so a finite maximum)
          const float f = fast_exp2(ms - mm);
          den = fmaf(f, ss.l(s2, g), den);
          num = fmaf(f, ss.acc(s2, g, d), num);
        }
      }
      const int64_t row = static_cast<int64_t>(pi ? pair_b : (pair ? pair_a : seq)) * a.o_sb;
      static_cast<T*>(a.out)[row + (h0 + g) * a.o_sh + d] = from_f32<T>(num / den);
    }
    return;
  }
  if constexpr (!PREFILL) {
    if (pair) {
      __syncthreads();
      // Wave w walked blocks [w * share, (w + 1) * share) of the two sequences laid end
      // to end: the first sequence's states are slot 0 of waves 0 .. wa - 1; the
      // second's are in waves wb .. W - 1, in slot 1 of a wave that also walked the first.
      const int W = a.wpg;
      const int wa = min((n_a + share - 1) / share, W), wb = n_a / share;
      const int parts = pair_b >= 0 ? 2 : 1;
      for (int t = threadIdx.x; t < parts * HT * D; t += W * kWave) {
        const int pi = t / (HT * D);
        const int g = (t % (HT * D)) / D, d = t % D;
        const int w0 = pi ? wb : 0, w1 = pi ? W : wa;
        float mm = kNoMax;
        for (int w = w0; w < w1; ++w) mm = fmaxf(mm, ss.m(2 * w + (pi && w * share < n_a), g));
        float den = 0.f, num = 0.f;
        for (int w = w0; w < w1; ++w) {
          const int sl = 2 * w + (pi && w * share < n_a);
          const float f = fast_exp2(ss.m(sl, g) - mm);
          den = fmaf(f, ss.l(sl, g), den);
          num = fmaf(f, ss.acc(sl, g, d), num);
        }
        const int64_t row = static_cast<int64_t>(pi ? pair_b : pair_a) * a.o_sb;
        static_cast<T*>(a.out)[row + (h0 + g) * a.o_sh + d] = from_f32<T>(num / den);
      }
      return;
    }
    if (a.wpg > 1) {
      merge_group_waves<T, D, HT>(a, ss, seq, h0, split, orow);
      return;
    }
  }
  if (tl != 0) return;

  if (PREFILL || a.splits == 1) {
    T* op = static_cast<T*>(a.out) + orow;
#pragma unroll
    for (int g = 0; g < HT; ++g) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        Pack16<T> o;
#pragma unroll
        for (int j = 0; j < VEC; ++j) o.v[j] = from_f32<T>(st.acc[g][i * VEC + j] / st.l[g]);
        store16(op + (h0 + g) * a.o_sh + (i * LPT + c) * VEC, o);
      }
    }
  } else {
#pragma unroll
    for (int g = 0; g < HT; ++g) {
      const int64_t part = (static_cast<int64_t>(seq) * a.Hq + h0 + g) * a.splits + split;
      if (c == 0) {
        a.m[part] = st.l[g] > 0.f ? st.m[g] : -INFINITY;
        a.l[part] = st.l[g];
      }
      float* ap = a.acc + part * D;
#pragma unroll
      for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int j = 0; j < VEC; j += 4)
          *reinterpret_cast<float4*>(ap + (i * LPT + c) * VEC + j) =
              make_float4(st.acc[g][i * VEC + j], st.acc[g][i * VEC + j + 1],
                          st.acc[g][i * VEC + j + 2], st.acc[g][i * VEC + j + 3]);
    }
  }
}

// Max over the 64 lanes of a wave; every lane ends with it.
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, xor_lane<1>(x));
  x = fmaxf(x, xor_lane<2>(x));
  x = fmaxf(x, xor_lane<4>(x));
  x = fmaxf(x, xor_lane<8>(x));
  x = fmaxf(x, xor_lane<16>(x));
  return halves_max(x);
}

// The split-K combine: one wave per (sequence, query head). Lane s holds split s's
// maximum and denominator (64 splits at a time) and the wave reduces them; then each lane
// owns output elements lane + 64 e and issues the partial-sum loads of 8 splits at once
// before accumulating them, so a (sequence, head) waits on memory a few times, not once
// per split and element.
template <typename T, int ED>
__global__ __launch_bounds__(64) void combine_kernel(const float* __restrict__ m,
                                                     const float* __restrict__ l,
                                                     const float* __restrict__ acc, T* out,
                                                     int Hq, int D, int64_t o_sb, int64_t o_sh,
                                                     int splits) {
  constexpr int kU = 8;  // splits whose loads are in flight together
  constexpr int kFew = 16;  // up to this many splits: every load issued at once
  const int lane = threadIdx.x;
  const int b = blockIdx.x, h = blockIdx.y;
  const int64_t base = (static_cast<int64_t>(b) * Hq + h) * splits;
  if (splits <= kFew) {
    // One round trip: the maxima, denominators and every partial sum are loaded before
    // any is used; then the same operations, in the same order, as the general path.
    const bool mine = lane < splits;
    const float mv = mine ? m[base + lane] : -INFINITY;
    const float lv = mine ? l[base + lane] : 0.f;
    float x[kFew][ED];
#pragma unroll
    for (int u = 0; u < kFew; ++u)
#pragma unroll
      for (int e = 0; e < ED; ++e) {
        const int d = lane + kWave * e;
        x[u][e] = u < splits && d < D ? acc[(base + u) * D + d] : 0.f;
      }
    __builtin_amdgcn_sched_barrier(0);
    const float mmax = wave_max(mv);
    const float wgt = mine ? fast_exp2(mv - mmax) : 0.f;
    const float den = group_sum<kWave>(mine ? fmaf(wgt, lv, 0.f) : 0.f);
    float num[ED];
#pragma unroll
    for (int e = 0; e < ED; ++e) num[e] = 0.f;
#pragma unroll
    for (int u = 0; u < kFew; ++u) {
      const float w = __shfl(wgt, u);  // 0 past the last split
#pragma unroll
      for (int e = 0; e < ED; ++e) num[e] = fmaf(w, x[u][e], num[e]);
    }
    T* op = out + b * o_sb + h * o_sh;
#pragma unroll
    for (int e = 0; e < ED; ++e) {
      const int d = lane + kWave * e;
      if (d < D) op[d] = from_f32<T>(num[e] / den);
    }
    return;
  }
  float mmax = -INFINITY;
  for (int s0 = 0; s0 < splits; s0 += kWave)
    if (s0 + lane < splits) mmax = fmaxf(mmax, m[base + s0 + lane]);
  mmax = wave_max(mmax);
  float den = 0.f;
  float num[ED];
#pragma unroll
  for (int e = 0; e < ED; ++e) num[e] = 0.f;
  for (int s0 = 0; s0 < splits; s0 += kWave) {
    const bool mine = s0 + lane < splits;
    const float wgt = mine ? fast_exp2(m[base + s0 + lane] - mmax) : 0.f;
    if (mine) den = fmaf(wgt, l[base + s0 + lane], den);
    const int n = min(kWave, splits - s0);
    for (int j = 0; j < n; j += kU) {
      float x[kU][ED];
#pragma unroll
      for (int u = 0; u < kU; ++u)
#pragma unroll
        for (int e = 0; e < ED; ++e) {
          const int d = lane + kWave * e;
          x[u][e] = j + u < n && d < D ? acc[(base + s0 + j + u) * D + d] : 0.f;
        }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const float w = __shfl(wgt, j + u);  // 0 past the last split
#pragma unroll
        for (int e = 0; e < ED; ++e) num[e] = fmaf(w, x[u][e], num[e]);
      }
    }
  }
  den = group_sum<kWave>(den);
  T* op = out + b * o_sb + h * o_sh;
#pragma unroll
  for (int e = 0; e < ED; ++e) {
    const int d = lane + kWave * e;
    if (d < D) op[d] = from_f32<T>(num[e] / den);
  }
}

template <typename T, int D, int HT, bool PREFILL>
static int launch_attend(const AttendArgs& a, dim3 grid, bool light, size_t lds, hipStream_t stream) {
  if constexpr (!PREFILL) {
    if (a.cuts > 1) {
      // In-workgroup split-K over the reference's split ranges (cut mode).
      if constexpr (D == 64 || D == 128) {
        if (light && a.stream_kv) {
          hipLaunchKernelGGL((paged_attend_kernel<T, D, HT, false, kLightStream, true>), grid,
                             dim3(kWave * a.wpg), lds, stream, a);
          return launch_status();
        }
      }
      if (light)
        hipLaunchKernelGGL((paged_attend_kernel<T, D, HT, false, kLight, true>), grid,
                           dim3(kWave * a.wpg), lds, stream, a);
      else
        hipLaunchKernelGGL((paged_attend_kernel<T, D, HT, false, kHeavy, true>), grid,
                           dim3(kWave * a.wpg), lds, stream, a);
      return launch_status();
    }
  }
  {
    if constexpr (!PREFILL && (D == 64 || D == 128)) {
      if (light && a.stream_kv) {
        hipLaunchKernelGGL((paged_attend_kernel<T, D, HT, PREFILL, kLightStream>), grid,
                           dim3(kWave * a.wpg), lds, stream, a);
        return launch_status();
      }
    }
    if (light) {
      hipLaunchKernelGGL((paged_attend_kernel<T, D, HT, PREFILL, kLight>), grid,
                         dim3(kWave * a.wpg), lds, stream, a);
      return launch_status();
    }
  }
  hipLaunchKernelGGL((paged_attend_kernel<T, D, HT, PREFILL, kHeavy>), grid, dim3(kWave * a.wpg),
                     lds, stream, a);
  return launch_status();
}

template <typename T, bool PREFILL>
static int dispatch_d(const AttendArgs& a, int D, int ht, dim3 grid, bool light, size_t lds,
                      hipStream_t stream) {
#define TS_HT(DD)                                                                \
  switch (ht) {                                                                  \
    case 1: return launch_attend<T, DD, 1, PREFILL>(a, grid, light, lds, stream); \
    case 2: return launch_attend<T, DD, 2, PREFILL>(a, grid, light, lds, stream); \
    case 4: return launch_attend<T, DD, 4, PREFILL>(a, grid, light, lds, stream); \
    default: return TS_EUNSUPPORTED;                                             \
  }
  switch (D) {
    case 8: TS_HT(8)
    case 16: TS_HT(16)
    case 32: TS_HT(32)
    case 64: TS_HT(64)
    case 128: TS_HT(128)
    case 256: TS_HT(256)
    default: break;
  }
#undef TS_HT
  return TS_EUNSUPPORTED;
}

// Launches of two or more rounds of one-wave-per-SIMD waves, or whose waves walk few
// tokens, take the light budget.
static bool light_budget(int64_t waves, bool short_walks) {
  return short_walks || waves >= 8 * static_cast<int64_t>(compute_units());
}

template <bool PREFILL>
static int dispatch_attend(const AttendArgs& a, int dtype, int D, int ht, dim3 grid,
                           bool light, size_t lds, hipStream_t stream) {
  switch (dtype) {
    case TS_F32: return dispatch_d<float, PREFILL>(a, D, ht, grid, light, lds, stream);
    case TS_F16: return dispatch_d<f16, PREFILL>(a, D, ht, grid, light, lds, stream);
    case TS_BF16: return dispatch_d<bf16, PREFILL>(a, D, ht, grid, light, lds, stream);
    default: return TS_EUNSUPPORTED;
  }
}

// Query heads one wave handles: 1 (per-head launch) or the GQA group, at most 4 (larger
// groups use several waves per kv head, each re-reading the kv head's blocks).
static int head_tile_for(int group, int head_tile) {
  if (head_tile == 1) return 1;
  if (head_tile != 0 || !is_pow2(group)) return -1;
  return group < 4 ? group : 4;
}

// The generic varlen prefill (fp32 or head dims without an MFMA kernel): one wave per
// (query row, head tile) running the decode loop over keys 0 .. its position.
int prefill_rows_generic(const void* q, const void* k, const void* v, void* out,
                         const int32_t* bt, const int32_t* q_starts, const int32_t* q_lens,
                         const int32_t* ctx_lens, int R, int Hq, int Hkv, int D, int lbs,
                         int max_q_len, int64_t q_st, int64_t q_sh, int64_t o_st, int64_t o_sh,
                         int64_t k_ss, int64_t k_sh, int64_t bt_s, float scale, int dtype,
                         hipStream_t stream) {
  const int group = Hq / Hkv;
  const int ht = head_tile_for(group, 0);
  if (ht < 0) return TS_EINVAL;
  AttendArgs a{q, k, v, bt, ctx_lens, out, nullptr, nullptr, nullptr, q_starts, q_lens,
               Hq, group, lbs, 1, 1, max_q_len, 0, 0, q_st, q_sh, o_st, o_sh, k_ss, k_sh, bt_s,
               scale * kLog2e};
  dim3 grid(static_cast<unsigned>(R) * max_q_len, Hq / ht, 1);
  const int64_t waves = static_cast<int64_t>(grid.x) * grid.y;
  return dispatch_attend<true>(a, dtype, D, ht, grid, light_budget(waves, false), 0, stream);
}

template <typename T>
static int launch_combine(const float* m, const float* l, const float* acc, T* out, int B, int Hq,
                          int D, int64_t o_sb, int64_t o_sh, int splits, hipStream_t st) {
  const dim3 grid(B, Hq);
  if (D <= kWave) {
    hipLaunchKernelGGL((combine_kernel<T, 1>), grid, dim3(kWave), 0, st, m, l, acc, out, Hq, D, o_sb, o_sh, splits);
  } else if (D <= 2 * kWave) {
    hipLaunchKernelGGL((combine_kernel<T, 2>), grid, dim3(kWave), 0, st, m, l, acc, out, Hq, D, o_sb, o_sh, splits);
  } else {
    hipLaunchKernelGGL((combine_kernel<T, 4>), grid, dim3(kWave), 0, st, m, l, acc, out, Hq, D, o_sb, o_sh, splits);
  }
  return launch_status();
}

}  // namespace ts

using namespace ts;

namespace ts {

// The launch shape of one decode call, from shapes only (never from lengths, so a
// captured graph always launches the same grid).
struct DecodePlan {
  int ht;         // query heads per wave
  int wpg;        // waves per workgroup
  int by_length;  // workgroups take length pairs
  int budget;     // kHeavy, kLight or kLightStream
  dim3 grid;
  size_t lds;     // dynamic LDS bytes
};

// Tokens one wave streams per loop iteration (TPW of the kernel's RowShape).
static int tokens_per_iteration(int dtype, int D, int ht, int budget) {
  const int lb = budget != kHeavy ? (ht == 4 ? 16 : 32) : 64;
  const int row = D * (dtype == TS_F32 ? 4 : 2);
  const int lpt = row <= lb ? 1 : std::min(row / lb, kWave);
  return kWave / lpt;
}

// LDS of a cut-mode workgroup: its pieces' states.
constexpr size_t kMaxInGroupLds = 64 << 10;

static int plan_decode(int B, int Hq, int Hkv, int D, int block_size, int max_blocks, int splits,
                       int head_tile, int dtype, DecodePlan* plan) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || splits < 1 || !is_pow2(block_size))
    return TS_EINVAL;
  const int group = Hq / Hkv;
  const int ht = head_tile_for(group, head_tile);
  if (ht < 0) return TS_EINVAL;
  const int64_t waves = static_cast<int64_t>(B) * (Hq / ht) * splits;
  const int64_t want = 4 * static_cast<int64_t>(compute_units());
  int wpg = 1;
  while (wpg < kMaxWavesPerGroup && waves * wpg * 2 <= want) wpg *= 2;
  // Up to 64 sequences whose workgroups are two-wave (one round of them fills the chip):
  // pair sequences by length instead, the longest with the shortest, in four-wave
  // workgroups. A batch of equal contexts runs exactly as before (two waves per
  // sequence); one of mixed lengths no longer waits on its longest sequences.
  int by_length = B <= kWave && B >= 2 && splits == 1 && wpg == 2 ? 1 : 0;
  if (by_length) wpg = kMaxWavesPerGroup;
  // The table width bounds the tokens a wave walks; waves of at most 256 tokens spend
  // much of their life in start-up and merge, which the light budget's second wave per
  // SIMD hides (measured: +6% to +43% up to 256 tokens a wave; -15% to +4% at 512;
  // -10% from 1024).
  const int64_t walk = static_cast<int64_t>(max_blocks) * block_size * (by_length ? 2 : 1) /
                       (static_cast<int64_t>(splits) * wpg);
  const int64_t grid_waves =
      static_cast<int64_t>(Hq / ht) * (by_length ? (B + 1) / 2 : B) * splits * wpg;
  // K/V (bounded by the table width) larger than the 256 MiB last-level cache: it is read
  // once, so it goes through non-temporal loads (caching it only evicts other lines), under
  // the light budget, in workgroups of up to 8 waves sized for one round of the chip
  // (8 waves per CU); length pairs then take 8 waves, so each sequence of a pair keeps
  // about 4. Measured against the heavy one-round launch: +13% to +16.5% at 64 x 4096
  // (189.6 -> 164.9 us, 6.5 TB/s), 32 x 4096, 64 x 2048, 16 x 8192 and 128 x 4096.
  // Smaller launches keep cached loads, which let K/V that a previous step left in the
  // cache be read from there (32 x 256: -13% with non-temporal loads). The non-temporal
  // instantiation exists for head rows of 64 and 128 elements only; other head dims keep
  // the cached policy.
  const int64_t kv_bytes = static_cast<int64_t>(B) * max_blocks * block_size * Hkv * D *
                           (dtype == TS_F32 ? 4 : 2) * 2;
  const bool stream_kv = max_blocks > 0 && (D == 64 || D == 128) && kv_bytes > (int64_t{256} << 20);
  // Tiles of four query heads stream 16 bytes per lane under the light budget; they run
  // the heavy budget instead (64 bytes per lane, three iterations in flight, one wave per
  // SIMD) with cached loads, which also let the second tile of a kv head's blocks (groups
  // of eight) read them from L2. Measured against the light streaming launch: 64 x 4096
  // with 32 / 8 heads 207 -> 193 us, 128 x 4096 407 -> 379 us, 64 / 8 heads 406 -> 328
  // us, 16 x 8192 bf16 208 -> 158 us; with non-temporal loads the heavy launch took
  // 212, 424, 426 and 186 us. Rows of 64 elements likewise (64 x 4096 130 -> 120 us,
  // 64 x 8192 257 -> 233 us); two-head tiles of 128-element rows keep the light budget
  // (the heavy one: 184 against 160 us at 64 x 4096).
  const bool heavy_stream = stream_kv && (ht == 4 || D == 64);
  if (stream_kv && by_length) wpg = heavy_stream ? kMaxWavesPerGroup : kMaxWavesLight;
  // Cached launches of two-head tiles of 16-bit 128- or 64-element rows: the light budget
  // at any walk length (measured against heavy: equal or faster on every shape from
  // 32 x 256 to 64 x 1024 and 24 x 2048, e.g. 64 x 1024 45.2 -> 42.1 us; D=64 64 x 1024
  // 26.4 -> 23.5 us, 128 x 1024 54.1 -> 44.4 us). Four-head tiles keep the rule below
  // (64 x 1024 with 32 / 8 heads: heavy 49.1, light 77.7 us).
  const bool light_rows = ht <= 2 && (D == 128 || D == 64) && dtype != TS_F32;
  const bool light = (stream_kv && !heavy_stream) ||
                     (!stream_kv && (light_rows || light_budget(grid_waves, max_blocks > 0 && walk < 512)));
  // With two waves per SIMD the chip holds twice the waves: up to 8 per workgroup, so
  // that each walks fewer tokens (fewer dependent rounds of loads per wave).
  if (stream_kv && !by_length && !heavy_stream) {
    while (wpg < kMaxWavesLight && waves * wpg < 2 * want) wpg *= 2;
  } else if (light && !by_length) {
    while (wpg < kMaxWavesLight && waves * wpg * 2 <= 2 * want) wpg *= 2;
  }
  plan->ht = ht;
  plan->wpg = wpg;
  plan->by_length = by_length;
  plan->budget = !light ? kHeavy : stream_kv ? kLightStream : kLight;
  plan->grid = dim3(Hq / ht, by_length ? (B + 1) / 2 : B, splits);
  // LDS: one merged state per wave (two per wave for a pair); none for one-wave groups.
  plan->lds = wpg > 1 ? static_cast<size_t>((by_length ? 2 : 1) * wpg * state_slot_bytes(ht, D)) : 0;
  return 0;
}

}  // namespace ts

extern "C" int ts_decode_plan(int B, int Hq, int Hkv, int D, int block_size, int max_blocks,
                              int splits, int head_tile, int dtype, int* out) {
  if (!out) return TS_EINVAL;
  DecodePlan p;
  const int rc = plan_decode(B, Hq, Hkv, D, block_size, max_blocks, splits, head_tile, dtype, &p);
  if (rc) return rc;
  out[0] = p.budget;
  out[1] = p.wpg;
  out[2] = p.by_length;
  out[3] = p.ht;
  out[4] = static_cast<int>(p.grid.x);
  out[5] = static_cast<int>(p.grid.y);
  out[6] = static_cast<int>(p.grid.z);
  out[7] = static_cast<int>(p.lds);
  return 0;
}

extern "C" int ts_decode_split(const void* q, const void* k_cache, const void* v_cache,
                               const int32_t* block_tables, const int32_t* context_lens,
                               void* out, float* m, float* l, float* acc, int B, int Hq,
                               int Hkv, int D, int block_size, int64_t q_stride_b,
                               int64_t q_stride_h, int64_t o_stride_b, int64_t o_stride_h,
                               int64_t k_stride_slot, int64_t k_stride_head, int64_t bt_stride,
                               int max_blocks, int splits, int head_tile, float scale, int dtype,
                               void* stream) {
  if (B < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || splits < 1 || !is_pow2(block_size))
    return TS_EINVAL;
  if (B == 0) return 0;
  if (B > 65535) return TS_EUNSUPPORTED;  // sequences are the grid's y dimension
  // m, l and acc all null with splits > 1: the split ranges stay inside each workgroup.
  const bool in_group = splits > 1 && !m && !l && !acc;
  if (splits > 1 && !in_group && (!m || !l || !acc)) return TS_EINVAL;
  if ((splits == 1 || in_group) && !out) return TS_EINVAL;
  DecodePlan p;
  const int rc = plan_decode(B, Hq, Hkv, D, block_size, max_blocks, in_group ? 1 : splits, head_tile,
                             dtype, &p);
  if (rc) return rc;
  AttendArgs a{q, k_cache, v_cache, block_tables, context_lens, out, m, l, acc, nullptr,
               nullptr, Hq, Hq / Hkv, ilog2(block_size), in_group ? 1 : splits, p.wpg, 0,
               p.by_length, B, q_stride_b, q_stride_h, o_stride_b, o_stride_h, k_stride_slot,
               k_stride_head, bt_stride, scale * kLog2e, 0};
  a.stream_kv = p.budget == kLightStream ? 1 : 0;
  a.width = max_blocks > 0 && max_blocks <= kWave && !p.by_length ? max_blocks : 0;
  size_t lds = p.lds;
  if (in_group) {
    // A piece ends at a split boundary between two loop iterations only if an
    // iteration's tokens never straddle a block; every piece's state needs an LDS slot.
    if (block_size % tokens_per_iteration(dtype, D, p.ht, p.budget)) return TS_EUNSUPPORTED;
    lds = static_cast<size_t>((p.by_length ? 2 : 1) * (splits + p.wpg) * state_slot_bytes(p.ht, D));
    if (lds > kMaxInGroupLds) return TS_EUNSUPPORTED;
    a.cuts = splits;
  }
  return dispatch_attend<false>(a, dtype, D, p.ht, p.grid, p.budget != kHeavy, lds,
                                static_cast<hipStream_t>(stream));
}

extern "C" int ts_decode_combine(const float* m, const float* l, const float* acc, void* out,
                                 int B, int Hq, int D, int64_t o_stride_b, int64_t o_stride_h,
                                 int splits, int dtype, void* stream) {
  if (B < 0 || Hq <= 0 || D <= 0 || splits < 1) return TS_EINVAL;
  if (B == 0) return 0;
  if (D > 4 * kWave) return TS_EUNSUPPORTED;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TS_F32: return launch_combine<float>(m, l, acc, static_cast<float*>(out), B, Hq, D, o_stride_b, o_stride_h, splits, st);
    case TS_F16: return launch_combine<f16>(m, l, acc, static_cast<f16*>(out), B, Hq, D, o_stride_b, o_stride_h, splits, st);
    case TS_BF16: return launch_combine<bf16>(m, l, acc, static_cast<bf16*>(out), B, Hq, D, o_stride_b, o_stride_h, splits, st);
    default: return TS_EUNSUPPORTED;
  }
}

// ---- the no-allocation variant ----------------------------------------------------------
// The split partials of ts_decode_attention_noalloc live in this array: one copy per
// device, held until the process ends. Host code never passes `scratch` itself (on the
// host it names a stand-in, not device memory): the device address of each device's copy
// is looked up once, with that device current, and kept.
namespace ts {
constexpr int64_t kNoAllocScratchFloats = TS_NOALLOC_SCRATCH_BYTES / sizeof(float);
}  // namespace ts

static __device__ __align__(256) float scratch[ts::kNoAllocScratchFloats];

namespace ts {

constexpr int kMaxScratchDevices = 64;
static std::atomic<float*> g_scratch_ptr[kMaxScratchDevices];
static std::mutex g_scratch_mu;

// Device address of the current device's scratch array (hipGetSymbolAddress on the first
// call per device). Returns 0 or a HIP error code.
static int current_scratch(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxScratchDevices) return TS_EUNSUPPORTED;
  float* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      void* addr = nullptr;
      e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return e;
      p = static_cast<float*>(addr);
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return 0;
}

}  // namespace ts

extern "C" int ts_decode_attention_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                           const int32_t* block_tables, const int32_t* context_lens,
                                           void* out, int B, int Hq, int Hkv, int D, int block_size,
                                           int64_t q_stride_b, int64_t q_stride_h,
                                           int64_t o_stride_b, int64_t o_stride_h,
                                           int64_t k_stride_slot, int64_t k_stride_head,
                                           int64_t bt_stride, int max_blocks, int splits,
                                           int head_tile, float scale, int dtype, void* stream) {
  if (B < 0 || Hq <= 0 || D <= 0 || splits < 1 || !out) return TS_EINVAL;
  if (splits > 1) {
    // acc [B, Hq, S, D] first (256-byte aligned, so its 16-byte stores stay aligned),
    // then m and l [B, Hq, S].
    const int64_t parts = static_cast<int64_t>(B) * Hq * splits;
    if (parts * (D + 2) > kNoAllocScratchFloats) return TS_ETOOBIG;
  }
  if (B == 0) return 0;
  if (splits == 1)
    return ts_decode_split(q, k_cache, v_cache, block_tables, context_lens, out, nullptr, nullptr,
                           nullptr, B, Hq, Hkv, D, block_size, q_stride_b, q_stride_h, o_stride_b,
                           o_stride_h, k_stride_slot, k_stride_head, bt_stride, max_blocks, 1,
                           head_tile, scale, dtype, stream);
  float* base = nullptr;
  const int rc = current_scratch(&base);
  if (rc) return rc;
  const int64_t parts = static_cast<int64_t>(B) * Hq * splits;
  float* acc = base;
  float* m = acc + parts * D;
  float* l = m + parts;
  // Every (sequence, head, split) partial is written by the split kernel (empty ranges as
  // m = -inf, l = 0, acc = 0), so nothing left by an earlier call is read.
  int e = ts_decode_split(q, k_cache, v_cache, block_tables, context_lens, out, m, l, acc, B, Hq,
                          Hkv, D, block_size, q_stride_b, q_stride_h, o_stride_b, o_stride_h,
                          k_stride_slot, k_stride_head, bt_stride, max_blocks, splits, head_tile,
                          scale, dtype, stream);
  if (e) return e;
  return ts_decode_combine(m, l, acc, out, B, Hq, D, o_stride_b, o_stride_h, splits, dtype, stream);
}

extern "C" int ts_version(void) { return (0 << 16) | 1; }

extern "C" const char* ts_strerror(int code) {
  if (code == 0) return "success";
  if (code == TS_EINVAL) return "invalid argument: sizes or strides do not fit together";
  if (code == TS_EUNSUPPORTED) return "unsupported shape or dtype: no compiled kernel";
  if (code == TS_ETOOBIG)
    return "the split partials exceed the no-allocation scratch (TS_NOALLOC_SCRATCH_BYTES per device)";
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "unknown error";
}
