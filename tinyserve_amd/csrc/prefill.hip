// Varlen causal prefill attention over the paged KV cache, on gfx950 MFMA.
//
// Reference behaviour: src/tinyserve/triton_prefill.py:50-125 (one program per
// (sequence, query tile, kv head), keys walked in chunks from position 0 to the tile's
// last query position, online softmax, P rounded to the value dtype before P.V) and
// src/tinyserve/attention.py:62-111 for the math it must equal.
//
// Work decomposition. A workgroup of 8 wave64s owns one kv head of one sequence and
// 32 * QB consecutive queries of HG of that kv head's query heads (HG * QB = 8): wave w
// takes query head hg = w % HG and the 32 queries of block qb = w / HG. All eight waves
// share each 64-key tile of K and V.
//
// Memory pipeline. K/V tiles are gathered from the paged cache (slot = table[pos / bs]
// * bs + pos % bs) straight into LDS with gfx950's direct-to-LDS loads
// (global_load_lds_dwordx4: lane l's 16 bytes land at the instruction's LDS base +
// 16 l), through a ring of three stages: while tile t is computed, tiles t + 1 and t + 2
// are in flight. No registers stage the data and no LDS store instructions are issued.
// One load instruction covers RPI consecutive keys (4 at D=128). When a cache block holds
// at least RPI slots those keys share one block, so the block id is a scalar load of the
// table and the address a scalar base plus a per-lane row/unit offset: the gather costs
// the VALU almost nothing. Smaller blocks take per-lane ids from a window of 512 table
// entries staged in LDS (refilled when a gather passes its end). Either way the
// vector-memory counter covers exactly the ring's loads and each stage is waited for with
// an exact vmcnt.
//
// Dispatch order. Workgroup b = (tile_rev * R + r) * heads + head: every sequence's last
// query tile (the one with the most keys) is dispatched, for all kv heads, before any
// earlier tile, so the long-running workgroups start first; and since the hardware
// deals workgroups to the 8 XCDs round-robin, with 8 kv heads each head's workgroups
// share one XCD's L2, where its K/V blocks are re-read by every query tile.
//
// Three shapes: 8 waves with a 3-stage ring of 64-key tiles (one workgroup per CU, 98 KB
// of LDS, two waves per SIMD) for large launches and prefix-hit chunks; for launches with
// too few query tiles to fill the chip that way (one or two prompts), 8 waves over the
// queries of the 4-wave shape (64 x 2 heads) with the keys split in two: waves w and
// w + 4 walk the lower and upper half of the key tiles (a 2-stage ring holding one tile
// of each half, 128 KB) and merge their softmax states through LDS at the end, which
// halves the longest workgroup's walk and puts two waves on each SIMD; and for mid-size
// launches, 4 waves over 32-key tiles (a 2-stage ring of 34 KB, 157 VGPRs: three
// workgroups, so three waves, per SIMD), whose extra wave per SIMD and finer key tiles
// outweigh the doubled barriers there. (Block sizes under 4 slots, 8 at D=64, run 4
// waves without the split: the halves' block ids come from the scalar-id gather.)
//
// MFMA formulation (v_mfma_f32_32x32x16_{f16,bf16}). Scores are computed transposed,
// S^T[key, query] = K . Q^T, with K as the A operand (one 16-byte LDS read per lane) and
// Q^T as the B operand (held in registers for the whole kernel). In the 32x32
// accumulator layout lane l holds column l % 32 -- one query -- and rows (keys)
// 8j + 4(l / 32) + i at item 4j + i, so each lane owns 16 of its query's scores per 32
// keys: the softmax max/sum are in-lane plus one exchange between the lane halves. The
// output is accumulated transposed too, O^T[d, query] += V^T . P^T: P^T is the B operand
// straight from the score registers (lane half h supplies keys {4h..4h+3, 8+4h..8+4h+3}
// of each 16-key chunk), and V^T is the A operand, read from the row-major V tile with
// two ds_read_b64_tr_b16 per MFMA. That instruction works on groups of 16 lanes: lane j
// of a group reads 4 consecutive 16-bit values ("row j") and lane i receives element
// i % 4 of rows i / 4, 4 + i / 4, 8 + i / 4, 12 + i / 4. Pointing lane j at
// V[key0 + j / 4][d0 + 4 (j % 4)] gives lane i the values V[key0 .. key0 + 3][d0 + i]:
// four keys of one d, the transposed operand.
//
// LDS layout: K and V tiles are [64 keys][D], rows unpadded, their 16-byte units
// XOR-swizzled per row (K by row & 15, V by a 4-row pattern), which keeps the K operand
// reads and the transposing V reads free of bank conflicts.
#include <algorithm>
#include <type_traits>

#include "common.h"

namespace ts {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));

#define TS_LDS __attribute__((address_space(3)))
#define TS_CONST __attribute__((address_space(4)))

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
  int n_kvh;
  int seq_group;  // > 0: dispatch in groups of this many sequences ranked by length
  int64_t q_st, q_sh, o_st, o_sh, k_ss, k_sh, bt_s;
  float scale_log2;
};

constexpr int kWin = 512;   // block ids held in LDS

template <int D, int W, int BN>
struct TileShape {
  static constexpr int kUPR = D / 8;          // 16-byte units per row
  static constexpr int kRPI = kWave / kUPR;   // rows one direct-to-LDS instruction fills
  static constexpr int kIPW = BN / kRPI / W;  // such instructions per wave per tensor
  static_assert(kIPW >= 1 && kIPW * kRPI * W == BN, "D in {64, 128}");
};

// Physical 16-byte unit of data unit u in row `row` of a tile is u ^ swz(row).
template <int D>
__device__ __forceinline__ int k_swz(int row) {
  return row & (D / 8 - 1);
}
template <int D>
__device__ __forceinline__ int v_swz(int row) {
  // 4-row patterns: {0, 6, 10, 12} for 16-unit rows, {0, 6, 4, 2} for 8-unit rows.
  constexpr uint32_t kTab = D == 128 ? 0x0C0A0600u : 0x02040600u;
  return (kTab >> ((row & 3) * 8)) & 0xFF;
}

// Instruction classes of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;

// One direct-to-LDS load of 16 bytes per lane (global_load_lds_dwordx4; M0 holds the
// LDS base). Issued as inline asm on purpose: the compiler's wait-count pass would
// otherwise guard every later LDS read with a wait for all such loads in flight (it
// cannot tell ring stages apart), draining the ring each step. The kernel orders these
// loads itself with counted waits before every ring barrier; loads the compiler does not
// count can only make its own waits stricter. Only the device pass sees the asm.
__device__ __forceinline__ void lds_load16(const void* src, TS_LDS void* dst) {
#if defined(__HIP_DEVICE_COMPILE__)
  // M0 is reserved to the compiler: the asm saves and restores it around the load.
  const uint32_t lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(dst));
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dwordx4 %2, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds), "v"(src)
      : "memory");
#endif
}

// The same load with a scalar base address and a 32-bit per-lane byte offset
// (global_load_lds_dwordx4 voffset, saddr): the address arithmetic of a gather whose
// lanes share one cache block stays on the scalar unit.
// M0 is bound through the asm operand, so the compiler sets it (one instruction) and
// knows it is taken.
__device__ __forceinline__ void lds_load16_s(const void* base, uint32_t voff, TS_LDS void* dst) {
#if defined(__HIP_DEVICE_COMPILE__)
  const uint32_t lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(dst));
  asm volatile("global_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(base), "{m0}"(lds) : "memory");
#endif
}

// Wait until at most N of this wave's vector-memory operations are in flight and all its
// LDS operations are done, then meet the other waves at s_barrier. __syncthreads() would
// also fence workgroup memory, which waits for every load in flight (vmcnt(0)) and so
// drains the ring; the tiles' visibility needs only each wave's own counted wait. The
// signal fences (no instructions) keep the compiler from moving memory accesses across.
template <int N>
__device__ __forceinline__ void ring_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt field");
  // vmcnt N (bits 3:0 and 15:14), expcnt 7 (no wait), lgkmcnt 0
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0070);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <typename T, int D, int HG, int QB, int kWaves, int kStages, int kBN, int kOcc,
          bool kScalarIds, int kParts>
__global__ __launch_bounds__(kWaves * kWave) __attribute__((amdgpu_waves_per_eu(kOcc, kOcc))) void
prefill_mfma_kernel(const PrefillArgs a) {
  using V8 = typename Mfma<T>::V8;
  // Key split (kParts > 1): waves w, w + kGW, ... take the same queries and heads; part
  // kh walks the kh-th contiguous share of the workgroup's key tiles, and the parts'
  // softmax states are merged through LDS at the end. kGW waves share a tile.
  constexpr bool kSplitK = kParts > 1;
  constexpr int kGW = kWaves / kParts;
  static_assert(kGW * kParts == kWaves, "whole waves per key part");
  static_assert(!kSplitK || (kScalarIds && kStages == 2), "key split: scalar ids, 2 stages");
  using Sh = TileShape<D, kGW, kBN>;
  constexpr int NH = kBN / 32;  // 32-key halves of S^T (one MFMA accumulator each)
  constexpr int NC = kBN / 16;  // 16-key chunks of P^T (one PV B operand each)
  static_assert(kStages == 2 || kStages == 3, "ring of 2 or 3 stages");
  constexpr int UPR = Sh::kUPR, RPI = Sh::kRPI, IPW = Sh::kIPW;
  constexpr int BQ = 32 * QB;
  constexpr int DT = D / 32;  // 32-row output tiles
  constexpr int KC = D / 16;  // 16-wide MFMA k-chunks of the head dim
  constexpr int TILE = kBN * D;
  constexpr int DMA_PER_TILE = 2 * IPW;  // direct-to-LDS instructions per wave per tile
  constexpr float kRescale = 8.0f;
  // bf16 keeps 8 significant bits: P rounded once would move outputs by up to ~1e-2
  // against the fp32 reference, so P is carried as hi + lo bf16 parts (about 16 bits)
  // and P.V takes two MFMAs. fp16's 11 bits meet the tolerance with one.
  constexpr bool kSplitP = std::is_same_v<T, bf16>;

  constexpr int kStageStride = kParts * TILE;  // one tile per key part
  __shared__ __attribute__((aligned(16))) T k_ring[kStages * kStageStride];
  __shared__ __attribute__((aligned(16))) T v_ring[kStages * kStageStride];
  __shared__ int32_t ids_lds[kWin];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kh = kSplitK ? wave / kGW : 0;           // key part
  const int wl = kSplitK ? wave - kh * kGW : wave;  // wave within its part
  const int col = lane & 31;  // this lane's query within the wave's 32
  const int half = lane >> 5;

  const int n_hc = a.n_kvh * a.hchunks;
  const int bid = blockIdx.x;
  const int rest = bid / n_hc;
  const int hcx = bid - rest * n_hc;
  int tile_rev, r;
  if (a.seq_group > 0) {
    // Groups of seq_group sequences of similar length, longest group first; within a
    // group, heaviest query tiles first. A group's K/V (one kv head per XCD) stays in
    // that XCD's L2 while its tiles run, which the plain order below loses when many
    // sequences are in flight at once. Lane b ranks sequence b by context length
    // (ties by index; R <= 64).
    const int per_group = a.n_qtiles * a.seq_group;
    const int gi = rest / per_group;
    const int rem = rest - gi * per_group;
    tile_rev = rem / a.seq_group;
    const int want = gi * a.seq_group + (rem - tile_rev * a.seq_group);
    if (want >= a.R) return;
    const int ln = threadIdx.x & (kWave - 1);
    const int mine = ln < a.R ? a.ctx_lens[ln] : -1;
    // Already in rank order (non-increasing lengths): no ranking loop.
    const int next = __shfl_down(mine, 1);
    int rank = ln;
    if (!__all(ln + 1 >= a.R || mine >= next)) {
      rank = 0;
      if (__all(mine < (1 << 25))) {
        // Unique keys (length, then lower index first): rank = keys above this one.
        const int key = ln < a.R ? mine * kWave + (kWave - 1 - ln) : -1;
        for (int j = 0; j < a.R; ++j) rank += __builtin_amdgcn_readlane(key, j) > key;
      } else {
        for (int j = 0; j < a.R; ++j) {
          const int other = __builtin_amdgcn_readlane(mine, j);
          rank += (other > mine) | ((other == mine) & (j < ln));
        }
      }
    }
    r = __builtin_ctzll(__ballot(ln < a.R && rank == want));
  } else {
    tile_rev = rest / a.R;
    r = rest - tile_rev * a.R;
  }
  const int q_len = a.q_lens[r];
  const int tile = (q_len + BQ - 1) / BQ - 1 - tile_rev;
  if (tile < 0) return;
  const int q0 = tile * BQ;
  const int ctx = a.ctx_lens[r];
  const int q_start = a.q_starts[r];
  const int kvh = hcx / a.hchunks;
  const int hc = hcx - kvh * a.hchunks;
  const int hg = wl % HG;
  const int qb = wl / HG;
  const int head = kvh * a.group + hc * HG + hg;
  const int past = ctx - q_len;  // position of query 0 is past + 0

  const int wq0 = q0 + qb * 32;
  const int qi = wq0 + col;
  const bool q_ok = qi < q_len;
  const int pos = past + qi;
  const int key_end = past + min(q0 + BQ, q_len);  // keys the workgroup needs
  const int key_last = key_end - 1;
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

  // Q is complete before the loop: without this wait the compiler re-checks the Q loads
  // with a full vmcnt(0) at every step, which would also wait for the ring's loads.
  __builtin_amdgcn_s_waitcnt(0x0070);

  f32x16 oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) oacc[dt] = f32x16{};
  float m_run = -1.0e30f;  // running max of scale*log2e*score; finite, so 2^(m_run - x) is 0
  float l_run = 0.f;       // this lane half's share of the softmax denominator

  // ---- the gather: one tile of K and V into a ring stage --------------------------------
  // Block ids of the keys [win_key0, win_key0 + kWin << lbs) sit in LDS, so a gather
  // reads its ids with LDS loads and the vector-memory counter sees only the ring's
  // loads. The window is refilled (with the ring drained) when a gather passes its end:
  // every kWin blocks, i.e. never below 8192 keys for 16-slot blocks.
  const int32_t* btrow = a.bt + static_cast<int64_t>(r) * a.bt_s;
  const int lbs = a.lbs;
  const int bs_mask = (1 << lbs) - 1;
  const int nblk = (key_end + bs_mask) >> lbs;  // blocks holding keys 0 .. key_end - 1
  int win_blk0 = 0;                              // first block id index in the window
  auto fill_window = [&](int blk0) {
    win_blk0 = blk0;
    for (int i = tid; i < kWin; i += kWaves * kWave) {
      const int j = min(blk0 + i, nblk - 1);
      ids_lds[i] = btrow[j];
    }
  };
  const T* kbase = static_cast<const T*>(a.k) + static_cast<int64_t>(kvh) * a.k_sh;
  const T* vbase = static_cast<const T*>(a.v) + static_cast<int64_t>(kvh) * a.k_sh;
  const int dma_row = lane / UPR;   // row within an instruction's RPI rows
  const int dma_unit = lane % UPR;  // physical unit this lane fills

  // Keys past key_end read key_last (finite, owned data): their scores are masked and
  // their V rows meet P = 0.
  //
  // kScalarIds (block size >= RPI): the RPI rows of one load lie in one cache block, so
  // its block id comes from a scalar load of the table (cached in the scalar cache), its
  // base address is scalar, and a lane adds only its row and 16-byte unit.
  const TS_CONST int32_t* bt_c = (const TS_CONST int32_t*)(btrow);
  const uint32_t k_ss_bytes = static_cast<uint32_t>(a.k_ss) * sizeof(T);
  const uint32_t row_bytes = static_cast<uint32_t>(dma_row) * k_ss_bytes;
  uint32_t kunit[IPW], vunit[IPW], rows_bytes[IPW];
#pragma unroll
  for (int m = 0; m < IPW; ++m) {
    const int row = (wl * IPW + m) * RPI + dma_row;
    kunit[m] = 16u * static_cast<uint32_t>(dma_unit ^ k_swz<D>(row));
    vunit[m] = 16u * static_cast<uint32_t>(dma_unit ^ v_swz<D>(row));
    rows_bytes[m] = static_cast<uint32_t>(m * RPI + dma_row) * k_ss_bytes;
  }
  // A wave's IPW * RPI rows of a tile share one block when blocks hold that many slots.
  const bool wave_block = (1 << lbs) >= IPW * RPI;
  auto gather = [&](T* k_lds, T* v_lds, int n0) {
    if constexpr (kScalarIds) {
      if (wave_block) {
        // One block id and one base for all of the wave's loads; rows past key_last
        // read key_last, which lies in the same block.
        const int kw = __builtin_amdgcn_readfirstlane(min(n0 + wl * IPW * RPI, key_last));
        const int blk = bt_c[kw >> lbs];
        const uint64_t boff = ((static_cast<uint64_t>(static_cast<uint32_t>(blk)) << lbs) +
                               static_cast<uint32_t>(kw & bs_mask)) * k_ss_bytes;
        const uint32_t lim = static_cast<uint32_t>(key_last - kw) * k_ss_bytes;
        const char* kb = reinterpret_cast<const char*>(kbase) + boff;
        const char* vb = reinterpret_cast<const char*>(vbase) + boff;
#pragma unroll
        for (int m = 0; m < IPW; ++m) {
          const int row0 = (wl * IPW + m) * RPI;
          const uint32_t voff = min(rows_bytes[m], lim);
          lds_load16_s(kb, voff + kunit[m], (TS_LDS void*)(k_lds + row0 * D));
          lds_load16_s(vb, voff + vunit[m], (TS_LDS void*)(v_lds + row0 * D));
        }
        return;
      }
      // Every id first (scalar loads issued together, one wait), then the loads.
      int key0[IPW], blk[IPW];
#pragma unroll
      for (int m = 0; m < IPW; ++m) {
        key0[m] = __builtin_amdgcn_readfirstlane(min(n0 + (wl * IPW + m) * RPI, key_last));
        blk[m] = bt_c[key0[m] >> lbs];
      }
#pragma unroll
      for (int m = 0; m < IPW; ++m) {
        const int row0 = (wl * IPW + m) * RPI;
        const uint64_t slot0 = (static_cast<uint64_t>(static_cast<uint32_t>(blk[m])) << lbs) +
                               static_cast<uint32_t>(key0[m] & bs_mask);
        const uint64_t boff = slot0 * k_ss_bytes;
        // Rows past key_last read key_last.
        const uint32_t voff = min(row_bytes, static_cast<uint32_t>(key_last - key0[m]) * k_ss_bytes);
        lds_load16_s(reinterpret_cast<const char*>(kbase) + boff, voff + kunit[m],
                     (TS_LDS void*)(k_lds + row0 * D));
        lds_load16_s(reinterpret_cast<const char*>(vbase) + boff, voff + vunit[m],
                     (TS_LDS void*)(v_lds + row0 * D));
      }
      return;
    }
#pragma unroll
    for (int m = 0; m < IPW; ++m) {
      const int row0 = (wl * IPW + m) * RPI;
      const int row = row0 + dma_row;
      const int key = min(n0 + row, key_last);
      const int blk = ids_lds[(key >> lbs) - win_blk0];
      const int64_t slot = (static_cast<int64_t>(blk) << lbs) + (key & bs_mask);
      const int64_t off = slot * a.k_ss;
      lds_load16(kbase + off + 8 * (dma_unit ^ k_swz<D>(row)), (TS_LDS void*)(k_lds + row0 * D));
      lds_load16(vbase + off + 8 * (dma_unit ^ v_swz<D>(row)), (TS_LDS void*)(v_lds + row0 * D));
    }
  };
  // Whether the ids of keys up to min(n0 + kBN, key_end) - 1 lie in the window.
  auto in_window = [&](int n0) {
    if constexpr (kScalarIds) return true;  // no window
    return ((min(n0 + kBN, key_end) - 1) >> lbs) < win_blk0 + kWin;
  };

  // ---- per-lane constants of the operand reads -------------------------------------------
  const int kphys = k_swz<D>(col);  // K rows col and col + 32 swizzle alike
  // This lane's K operand of 16-wide chunk kc: row col, 16-byte unit (2 kc + half)
  // swizzled; the whole offset is kept per chunk, so a read is one address register plus
  // an immediate (stage and 32-key part).
  int kofs[KC];
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) kofs[kc] = col * D + ((2 * kc + half) ^ kphys) * 8;
  // V^T operand: lane j of its 16-lane group points at V[key0 + j / 4][d0 + 4 (j % 4)].
  const int vj = lane & 15;
  const int vdsub = (lane >> 4) & 1;
  const int vkey_lane = 4 * half + (vj >> 2);     // + 16 c0 + 8 t
  const int vd_lane = 16 * vdsub + 4 * (vj & 3);  // + 32 dt
  const int vswz = v_swz<D>(vkey_lane);           // key & 3 = vj >> 2 for every read

  auto attend = [&](const T* k_lds, const T* v_lds, int n0) __attribute__((always_inline)) {
    // S^T = K . Q^T for the tile's 32-key parts: NH independent MFMA chains. The K
    // operands of chunk kc + 1 are read while chunk kc multiplies.
    f32x16 s[NH];
#pragma unroll
    for (int h = 0; h < NH; ++h) s[h] = f32x16{};
    {
      auto kread = [&](int kc, V8 (&x)[NH]) {
#pragma unroll
        for (int h = 0; h < NH; ++h) x[h] = *reinterpret_cast<const V8*>(k_lds + kofs[kc] + 32 * h * D);
      };
      V8 ka[2][NH];
      kread(0, ka[0]);
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        if (kc + 1 < KC) kread(kc + 1, ka[(kc + 1) & 1]);
#pragma unroll
        for (int h = 0; h < NH; ++h) s[h] = Mfma<T>::mma(ka[kc & 1][h], qreg[kc], s[h]);
      }
      // Keep that order through scheduling: reads of chunk kc + 1, then MFMAs of kc.
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, NH, 0);
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        if (kc + 1 < KC) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, NH, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, NH, 0);
      }
    }
    // Causal mask, only on a tile that crosses this wave's diagonal: item v of part h
    // holds key n0 + 32 h + 8 (v / 4) + 4 half + v % 4.
    if (n0 + kBN - 1 > wave_pos_min) {
      const int lim = pos - n0 - 4 * half;
#pragma unroll
      for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          if (32 * h + 8 * (v >> 2) + (v & 3) > lim) s[h][v] = -INFINITY;
    }

    // Online softmax for this lane's query, in base 2 with the scale folded into one
    // FMA: p = 2^(s * c - m), c = scale * log2(e) > 0.
    const float c = a.scale_log2;
    V8 pk[NC];
    V8 pk_lo[kSplitP ? NC : 1];
    typedef float F2 __attribute__((ext_vector_type(2)));
    typedef T T2 __attribute__((ext_vector_type(2)));
    typedef T T4 __attribute__((ext_vector_type(4)));
    // P^T of the tile against the running maximum m_run; returns this lane's sum of P.
    auto make_p = [&]() -> float {
      const float neg_m = -m_run;
      float psum = 0.f;
#pragma unroll
      for (int c0 = 0; c0 < NC; ++c0) {
        const f32x16& sv = s[c0 >> 1];
        T2 h[4], lo[4];
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          const int v = 8 * (c0 & 1) + 2 * e2;
          const F2 pf = {fast_exp2(fmaf(sv[v], c, neg_m)), fast_exp2(fmaf(sv[v + 1], c, neg_m))};
          h[e2] = __builtin_convertvector(pf, T2);
          if constexpr (kSplitP) {
            psum += pf[0] + pf[1];
            lo[e2] = __builtin_convertvector(pf - __builtin_convertvector(h[e2], F2), T2);
          } else {
            // The denominator sums the rounded P that P.V uses: one v_dot2 per pair.
            psum = __builtin_amdgcn_fdot2(h[e2], T2{T(1), T(1)}, psum, false);
          }
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
      return psum;
    };
    // Lazy rescaling without a maximum on the common path: P is first computed against
    // the old running maximum. A lane's sum bounds each of its P, so if no lane's sum
    // exceeds 2^kRescale every P is at most 2^kRescale (exact in fp32, representable in
    // fp16/bf16) and the tile is done. Otherwise (whenever the scores grew by more than
    // kRescale) the exact maximum is taken, O and l are rescaled, and P is recomputed. A
    // wave's first tile (n0 == 0 for every wave) starts from the exact maximum, so it
    // needs no second pass: every row has a key there (key 0), so the maximum is finite.
    auto tile_max = [&]() -> float {
      float mx = s[0][0];
#pragma unroll
      for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int v = (h == 0 ? 1 : 0); v < 16; ++v) mx = fmaxf(mx, s[h][v]);
      return halves_max(mx) * c;
    };
    if (n0 == 0) m_run = tile_max();
    float psum = make_p();
    if (__any(!(psum <= exp2f(kRescale)))) {
      const float m_new = fmaxf(m_run, tile_max());
      const float alpha = fast_exp2(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
      m_run = m_new;
      psum = make_p();
    }
    l_run += psum;

    // O^T += V^T . P^T, the V^T operand by two transposing reads per MFMA; the operand
    // of step i + 1 is read while step i multiplies (step i = (dt, c0), c0 fastest).
    auto vread = [&](int i) -> V8 {
      const int dt = i / NC, c0 = i % NC;
      const int d = dt * 32 + vd_lane;
      s16x4 part[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int key = 16 * c0 + 8 * t + vkey_lane;
        const T* p = v_lds + key * D + (((d >> 3) ^ vswz) << 3) + (d & 7);
        part[t] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((TS_LDS s16x4*)(p));
      }
      return __builtin_bit_cast(V8, __builtin_shufflevector(part[0], part[1], 0, 1, 2, 3, 4, 5, 6, 7));
    };
    V8 va[2];
    va[0] = vread(0);
#pragma unroll
    for (int i = 0; i < NC * DT; ++i) {
      if (i + 1 < NC * DT) va[(i + 1) & 1] = vread(i + 1);
      const int dt = i / NC, c0 = i % NC;
      oacc[dt] = Mfma<T>::mma(va[i & 1], pk[c0], oacc[dt]);
      if constexpr (kSplitP) oacc[dt] = Mfma<T>::mma(va[i & 1], pk_lo[c0], oacc[dt]);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 1);
#pragma unroll
    for (int i = 0; i < NC * DT; ++i) {
      if (i + 1 < NC * DT) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 1);
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, kSplitP ? 2 : 1, 1);
    }
  };

  // ---- the ring: tile t lives in stage t % kStages --------------------------------------
  // Before computing tile t a wave waits for its own loads of tile t (with three stages
  // the loads of tile t + 1, if issued, may stay in flight), then the barrier makes every
  // wave's loads of tile t visible and certifies that all waves finished tile t - 1,
  // whose stage receives tile t + kStages - 1. Stage indices are compile-time constants
  // (the loop is unrolled kStages times), so every LDS address is a base plus an offset.
  auto step = [&](const T* k_cur, const T* v_cur, T* k_nx, T* v_nx, int n0) {
    if constexpr (kStages == 3) {
      if (n0 + kBN < key_end) ring_barrier<DMA_PER_TILE>();
      else ring_barrier<0>();
    } else {
      ring_barrier<0>();
    }
    const int nn = n0 + (kStages - 1) * kBN;
    if (nn < key_end) {
      if (!in_window(nn)) {  // rare: drain, move the window to the gather's first block
        __builtin_amdgcn_s_waitcnt(0x0070);
        __syncthreads();
        fill_window(nn >> lbs);
        __syncthreads();
      }
      gather(k_nx, v_nx, nn);
    }
    if (n0 < wave_key_end) attend(k_cur, v_cur, n0);
  };
  // Stage s of this wave's key part: one tile, at (s * kParts + kh) tiles.
  T* const k0 = k_ring + kh * TILE;
  T* const v0 = v_ring + kh * TILE;
  T* const k1 = k0 + kStageStride;
  T* const v1 = v0 + kStageStride;
  T* const k2 = k0 + (kStages - 1) * kStageStride;  // == k1 with two stages (never used)
  T* const v2 = v0 + (kStages - 1) * kStageStride;

  if constexpr (!kScalarIds) {
    fill_window(0);
    __syncthreads();
  }
  if constexpr (kSplitK) {
    // Part kh takes tiles kh * n_lo .. (kh + 1) * n_lo - 1 (the last part the rest); all
    // parts step n_lo times (the same barriers), later parts' last steps possibly with no
    // tile.
    const int ntiles = (key_end + kBN - 1) / kBN;
    const int n_lo = (ntiles + kParts - 1) / kParts;
    const int base = kh * n_lo * kBN;
    const int half_end = kh == kParts - 1 ? key_end : min((kh + 1) * n_lo * kBN, key_end);
    auto sstep = [&](const T* k_cur, const T* v_cur, T* k_nx, T* v_nx, int n0) {
      ring_barrier<0>();
      if (n0 + kBN < half_end) gather(k_nx, v_nx, n0 + kBN);
      if (n0 < half_end && n0 < wave_key_end) attend(k_cur, v_cur, n0);
    };
    if (base < half_end) gather(k0, v0, base);
    for (int i = 0; i < n_lo; i += 2) {
      sstep(k0, v0, k1, v1, base + i * kBN);
      if (i + 1 >= n_lo) break;
      sstep(k1, v1, k0, v0, base + (i + 1) * kBN);
    }
  } else {
  gather(k0, v0, 0);
  if constexpr (kStages == 3) {
    if (kBN < key_end) gather(k1, v1, kBN);
    for (int n0 = 0; n0 < key_end; n0 += 3 * kBN) {
      step(k0, v0, k2, v2, n0);
      if (n0 + kBN >= key_end) break;
      step(k1, v1, k0, v0, n0 + kBN);
      if (n0 + 2 * kBN >= key_end) break;
      step(k2, v2, k1, v1, n0 + 2 * kBN);
    }
  } else {
    for (int n0 = 0; n0 < key_end; n0 += 2 * kBN) {
      step(k0, v0, k1, v1, n0);
      if (n0 + kBN >= key_end) break;
      step(k1, v1, k0, v0, n0 + kBN);
    }
  }
  }
  // No load may still be writing this workgroup's LDS when its waves end.
  __builtin_amdgcn_s_waitcnt(0x0070);

  if constexpr (kSplitK) {
    // Merge every later part's state into part 0's, lane by lane (the waves have the same
    // layout), one part at a time: m, l and O^T[0] through k_ring, O^T[1..] through
    // v_ring, lane-fastest so that the accesses are conflict-free. Scores are in base-2
    // units.
    static_assert(kGW * (2 + 16) * kWave * 4 <= sizeof(k_ring), "parked m, l, O^T[0] fit");
    static_assert(kGW * (DT - 1) * 16 * kWave * 4 <= sizeof(v_ring), "parked O^T[1..] fit");
    float* xk = reinterpret_cast<float*>(k_ring) + wl * (2 + 16) * kWave + lane;
    float* xv = reinterpret_cast<float*>(v_ring) + wl * (DT - 1) * 16 * kWave + lane;
#pragma unroll
    for (int part = kParts - 1; part >= 1; --part) {
      __syncthreads();  // every wave is done with the ring (or with the previous merge)
      if (kh == part) {
        xk[0] = m_run;
        xk[kWave] = l_run;
#pragma unroll
        for (int e = 0; e < 16; ++e) xk[(2 + e) * kWave] = oacc[0][e];
#pragma unroll
        for (int dt = 1; dt < DT; ++dt)
#pragma unroll
          for (int e = 0; e < 16; ++e) xv[((dt - 1) * 16 + e) * kWave] = oacc[dt][e];
      }
      __syncthreads();
      if (kh == 0) {
        const float m1 = xk[0];
        const float mn = fmaxf(m_run, m1);
        const float a0 = fast_exp2(m_run - mn), a1 = fast_exp2(m1 - mn);
        l_run = l_run * a0 + xk[kWave] * a1;
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[0][e] = oacc[0][e] * a0 + xk[(2 + e) * kWave] * a1;
#pragma unroll
        for (int dt = 1; dt < DT; ++dt)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            oacc[dt][e] = oacc[dt][e] * a0 + xv[((dt - 1) * 16 + e) * kWave] * a1;
        m_run = mn;
      }
    }
    if (kh != 0) return;
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

// KP > 1: the key-split shape (W waves, W / KP per key part); its caller checks that the
// block size allows the scalar-id gather.
template <typename T, int D, int HG, int W, int S, int BN, int OCC, int KP = 1>
static int launch_prefill_mfma(const PrefillArgs& a, int Hkv, hipStream_t stream) {
  constexpr int QB = W / KP / HG;
  const int seqs = a.seq_group > 0 ? (a.R + a.seq_group - 1) / a.seq_group * a.seq_group : a.R;
  dim3 grid(static_cast<unsigned>(a.n_qtiles) * seqs * Hkv * a.hchunks);
  if constexpr (KP > 1) {
    hipLaunchKernelGGL((prefill_mfma_kernel<T, D, HG, QB, W, S, BN, OCC, true, KP>), grid,
                       dim3(W * kWave), 0, stream, a);
  } else {
    // A load's RPI rows share a cache block when blocks hold at least RPI slots.
    if ((1 << a.lbs) >= TileShape<D, W, BN>::kRPI)
      hipLaunchKernelGGL((prefill_mfma_kernel<T, D, HG, QB, W, S, BN, OCC, true, 1>), grid, dim3(W * kWave), 0, stream, a);
    else
      hipLaunchKernelGGL((prefill_mfma_kernel<T, D, HG, QB, W, S, BN, OCC, false, 1>), grid, dim3(W * kWave), 0, stream, a);
  }
  return launch_status();
}

// Query tiles of 32 * (W / HG) queries. The 8-wave shape is the faster one per unit of
// work; the 4-wave shape halves the work per workgroup and fits two workgroups per CU,
// which wins when the launch has fewer than two 8-wave workgroups per CU (e.g. one
// 2048-token prompt: 128 workgroups of 8 waves).
template <typename T, int D, int W, int S, int BN, int OCC, int KP = 1>
static int dispatch_hg_w(PrefillArgs& a, int Hkv, int max_q_len, int64_t n_rows, hipStream_t stream) {
  constexpr int WQ = W / KP;  // waves over the queries and heads
  const int hg = a.group < WQ ? a.group : WQ;
  a.hchunks = a.group / hg;
  const int bq = 32 * (WQ / hg);
  a.n_qtiles = (max_q_len + bq - 1) / bq;
  a.n_kvh = Hkv;
  // Length-ranked groups of 4096 / (mean new tokens) sequences (1 to 8, at most R: a
  // group's K/V about fits one XCD's L2), for 8-16 sequences, short prompts (mean up to
  // 512 new tokens), or 32 or more prompts of one length, up to 64 sequences; pairs for
  // 17-64 prompts of mixed lengths above that mean. Measured at Qwen3 shapes: +43% on 8
  // mixed prompts, +27% on 64 x 256, +5% on 16 x 512, +4-6% on 48-64 x 1024, +2% on
  // 32 x 2048, +5.6% on average (-0.4% to +24%) over 16 batches of 24-64 mixed prompts;
  // for a few long prompts (-2.6% at 4 x 2048; -7 to -12% for 4 equal ones) the plain
  // order is kept.
  a.seq_group = 0;
  if (a.R > 1 && a.R <= kWave && n_rows > 0) {
    const int64_t mean = (n_rows + a.R - 1) / a.R;
    const bool uniform = n_rows == static_cast<int64_t>(a.R) * max_q_len;
    if (a.R > 16 && !uniform && mean > 512) {
      a.seq_group = 2;
    } else if ((a.R >= 8 && a.R <= 16) || mean <= 512 || (uniform && a.R >= 32)) {
      const int g = static_cast<int>(std::min<int64_t>(8, std::max<int64_t>(1, 4096 / std::max<int64_t>(mean, 1))));
      a.seq_group = g < a.R ? g : a.R;
    }
  }
  switch (hg) {
    case 1: return launch_prefill_mfma<T, D, 1, W, S, BN, OCC, KP>(a, Hkv, stream);
    case 2: return launch_prefill_mfma<T, D, 2, W, S, BN, OCC, KP>(a, Hkv, stream);
    case 4:
      if constexpr (WQ >= 4) return launch_prefill_mfma<T, D, 4, W, S, BN, OCC, KP>(a, Hkv, stream);
      return TS_EUNSUPPORTED;
    case 8:
      if constexpr (WQ >= 8) return launch_prefill_mfma<T, D, 8, W, S, BN, OCC, KP>(a, Hkv, stream);
      return TS_EUNSUPPORTED;
    default: return TS_EUNSUPPORTED;
  }
}

// Which of the three workgroup shapes a launch runs (see the header comment). wg8 is the
// 8-wave grid. Measured at Qwen3 shapes: chunks of at most 128 new tokens (prefix hits)
// run the 8-wave shape (+2.5-9.5%); grids under 1.5 8-wave workgroups per CU (one or two
// long prompts) the 4-wave, 64-key shape at two per CU; grids of 1.5 to 8 per CU (3-16
// prompts of 2048, 1-4 of 4096-8192: +1-10%), and of up to 16 per CU when the mean new
// tokens per sequence is at most 1280 (8-32 mixed prompts, 16 x 512, 64 x 256: +5-14%),
// the 4-wave, 32-key shape at three per CU; larger grids the 8-wave shape.
enum class PrefillShape { kW8, kW4, kW4Short };

static PrefillShape prefill_shape(int R, int group, int Hkv, int max_q_len, int64_t n_rows) {
  const int hg8 = group < 8 ? group : 8;
  const int64_t wg8 = static_cast<int64_t>((max_q_len + 32 * (8 / hg8) - 1) / (32 * (8 / hg8))) *
                      R * Hkv * (group / hg8);
  const int64_t cus = compute_units();
  if (group > 4) return PrefillShape::kW8;
  // Up to 64 new tokens per sequence in a launch of at most half an 8-wave workgroup per
  // CU: the key-split shape (its 64 queries hold each sequence, and it halves every walk
  // of the long cached prefix; +5-25% there, -4% to -11% in larger launches).
  if (max_q_len <= 64 && 2 * wg8 <= cus) return PrefillShape::kW4;
  // Up to 128 new tokens per sequence: one 8-wave query tile holds a whole sequence, so
  // its K/V (the whole cached prefix) is read once per kv head, not once per 64 queries.
  if (max_q_len <= 128) return PrefillShape::kW8;
  if (2 * wg8 < 3 * cus) return PrefillShape::kW4;
  const bool short_mean = n_rows > 0 && n_rows <= 1280 * static_cast<int64_t>(R);
  if (wg8 <= 8 * cus || (short_mean && wg8 <= 16 * cus)) return PrefillShape::kW4Short;
  return PrefillShape::kW8;
}

template <typename T, int D>
static int dispatch_hg(PrefillArgs& a, int Hkv, int max_q_len, int64_t n_rows, hipStream_t stream) {
  switch (prefill_shape(a.R, a.group, Hkv, max_q_len, n_rows)) {
    case PrefillShape::kW4Short: return dispatch_hg_w<T, D, 4, 2, 32, 3>(a, Hkv, max_q_len, n_rows, stream);
    case PrefillShape::kW4:
      // Two key halves per workgroup (8 waves, one workgroup and two waves per SIMD per
      // CU) where the scalar-id gather applies; else the plain 4-wave shape.
      if ((1 << a.lbs) >= TileShape<D, 4, 64>::kRPI)
        return dispatch_hg_w<T, D, 8, 2, 64, 2, 2>(a, Hkv, max_q_len, n_rows, stream);
      return dispatch_hg_w<T, D, 4, 2, 64, 2>(a, Hkv, max_q_len, n_rows, stream);
    default: return dispatch_hg_w<T, D, 8, 3, 64, 2>(a, Hkv, max_q_len, n_rows, stream);
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
                                 int block_size, int max_q_len, int64_t n_rows,
                                 int64_t q_stride_t,
                                 int64_t q_stride_h, int64_t o_stride_t, int64_t o_stride_h,
                                 int64_t k_stride_slot, int64_t k_stride_head,
                                 int64_t bt_stride, float scale, int dtype, void* stream) {
  if (R < 0 || max_q_len < 0 || n_rows < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || !is_pow2(Hq / Hkv) ||
      !is_pow2(block_size))
    return TS_EINVAL;
  if (R == 0 || max_q_len == 0) return 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int lbs = ilog2(block_size);
  // The direct-to-LDS gather moves 16-byte units: rows must start 16-byte aligned.
  const bool aligned = (k_stride_slot % 8 == 0) && (k_stride_head % 8 == 0) &&
                       (reinterpret_cast<uintptr_t>(k_cache) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(v_cache) % 16 == 0);
  if ((dtype == TS_F16 || dtype == TS_BF16) && (D == 64 || D == 128) && aligned) {
    PrefillArgs a{q, k_cache, v_cache, out, block_tables, q_starts, q_lens, context_lens,
                  R, Hq / Hkv, 1, lbs, 1, Hkv, 0, q_stride_t, q_stride_h, o_stride_t, o_stride_h,
                  k_stride_slot, k_stride_head, bt_stride, scale * kLog2e};
    if (dtype == TS_F16) {
      return D == 64 ? dispatch_hg<f16, 64>(a, Hkv, max_q_len, n_rows, st)
                     : dispatch_hg<f16, 128>(a, Hkv, max_q_len, n_rows, st);
    }
    return D == 64 ? dispatch_hg<bf16, 64>(a, Hkv, max_q_len, n_rows, st)
                   : dispatch_hg<bf16, 128>(a, Hkv, max_q_len, n_rows, st);
  }
  return prefill_rows_generic(q, k_cache, v_cache, out, block_tables, q_starts, q_lens,
                              context_lens, R, Hq, Hkv, D, lbs, max_q_len, q_stride_t,
                              q_stride_h, o_stride_t, o_stride_h, k_stride_slot,
                              k_stride_head, bt_stride, scale, dtype, st);
}
