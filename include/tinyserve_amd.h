/*
 * tinyserve_amd.h: the C ABI of libtinyserve_amd.so, the MI355X (gfx950) kernels of
 * TinyServe's attention hot path.
 *
 * Every entry point takes plain device pointers, element strides and sizes, launches
 * on the given HIP stream (a hipStream_t passed as void*; NULL = the null stream) and
 * returns without synchronising, so each call may be captured into a HIP graph. The
 * library never allocates device memory: outputs and split-K partials are owned by the
 * caller. Return value: 0 on success, a negative TS_E* code for an argument the kernels
 * cannot take (nothing was launched), or a positive hipError_t from the launch.
 *
 * Strides are in ELEMENTS of the tensor they describe. The last (head_dim) dimension of
 * every tensor must be contiguous. Layouts follow the reference:
 *   q / out (decode)   [B, Hq, D]            (stride_b, stride_h, 1)
 *   q / out (prefill)  [T, Hq, D]            (stride_t, stride_h, 1)
 *   k_cache, v_cache   [num_slots, Hkv, D]   one layer; (stride_slot, stride_head, 1)
 *   block_tables       [B or R, W] int32     row stride bt_stride
 *   slot of position p = block_tables[row, p / block_size] * block_size + p % block_size
 *
 * Device-resident inputs are trusted, as the kernels cannot check them without a host
 * sync. The caller guarantees what the reference's Python checks before its launches
 * (check_decode_args, triton_attention.py:361-391; paged_prefill_attention,
 * triton_prefill.py:177-194):
 *   - every context length is at least 1, and the table row holds every block it
 *     covers, each a valid block of the cache;
 *   - for prefill, 0 <= q_lens[r] <= min(context_lens[r], max_q_len) (a sequence with
 *     no new rows is skipped), and rows
 *     q_starts[r] .. q_starts[r] + q_lens[r] - 1 exist in q and out;
 *   - slots passed to ts_qk_norm_rope_store lie in the cache.
 * Inputs outside these ranges make the kernels read or write out of bounds.
 */
#ifndef TINYSERVE_AMD_H
#define TINYSERVE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types. */
enum ts_dtype { TS_F32 = 0, TS_F16 = 1, TS_BF16 = 2 };

/* Negative return codes (argument errors, detected before any launch). */
#define TS_EINVAL (-1)      /* sizes or strides that do not fit together */
#define TS_EUNSUPPORTED (-2) /* a shape/dtype combination with no compiled kernel */
#define TS_ETOOBIG (-3)      /* ts_decode_attention_noalloc: partials beyond its scratch */

/* Library version, (major << 16) | minor. */
int ts_version(void);

/* Text for a return code of any entry point. */
const char* ts_strerror(int code);

/*
 * Paged GQA decode attention, one pass of split-K.
 *
 * Replaces the launches of _paged_decode_kernel, _paged_decode_grouped_kernel and
 * _paged_decode_split_kernel (reference src/tinyserve/triton_attention.py:76, :193,
 * :243), issued by launch_paged_decode (:394), launch_paged_decode_grouped (:447) and
 * launch_paged_decode_split (:534).
 *
 * One wavefront per (sequence, tile of `head_tile` query heads, split). Query head h reads
 * kv head h / (Hq / Hkv). head_tile = 1 is the per-query-head launch shape of
 * _paged_decode_kernel (any Hq / Hkv); head_tile = 0 picks the whole GQA group (it
 * needs Hq / Hkv to be a power of 2).
 *
 * Sequence b's blocks 0 .. ceil(lens[b] / block_size) - 1 are cut into `splits`
 * contiguous ranges of ceil(nblocks / splits) blocks (the reference's ranges,
 * triton_attention.py:283-286). splits == 1: `out` [B, Hq, D] receives the normalised
 * result in the q dtype and m/l/acc are not touched (may be NULL). splits > 1 with m, l
 * and acc all NULL: each (sequence, head tile) workgroup keeps every range's softmax state
 * in LDS, merges them by ts_decode_combine's rule and writes `out` (one launch, the
 * combine of _merge_splits_kernel, :299-327, included); TS_EUNSUPPORTED, before any
 * launch, if block_size is smaller than the tokens one loop iteration streams (16 at
 * fp16 D=128) or the states exceed 64 KiB of LDS, and the caller then takes the path
 * below. splits > 1 with m, l, acc: every range writes its fp32 partial to
 * m, l [B, Hq, splits] and acc [B, Hq, splits, D] (contiguous, part index
 * (b * Hq + h) * splits + split); `out` is not touched, and ts_decode_combine finishes the
 * result. m is stored in base-2 units (log2 e * max score).
 *
 * max_blocks: the width of block_tables (entries per row the caller filled, so every
 * context is at most max_blocks * block_size), or 0 if unknown. It only picks how the
 * launch runs: the register budget (short walks per wave run two waves per SIMD) and,
 * when the K/V it bounds exceeds 256 MiB (head dims 64 and 128), non-temporal K/V loads
 * with one round of two-wave-per-SIMD workgroups. Nothing is read by it, and a wrong
 * value costs speed, never correctness. Pass the tightest width known: a table padded to
 * the model's maximum position (a graph captured for any context) bounds far more K/V
 * than it holds, so every such launch takes the streaming shape, even at short contexts.
 * (The reference passes the table to Triton and has no such argument.)
 */
int ts_decode_split(const void* q, const void* k_cache, const void* v_cache,
                    const int32_t* block_tables, const int32_t* context_lens, void* out,
                    float* m, float* l, float* acc, int B, int Hq, int Hkv, int D,
                    int block_size, int64_t q_stride_b, int64_t q_stride_h,
                    int64_t o_stride_b, int64_t o_stride_h, int64_t k_stride_slot,
                    int64_t k_stride_head, int64_t bt_stride, int max_blocks, int splits,
                    int head_tile, float scale, int dtype, void* stream);

/*
 * The launch shape ts_decode_split picks for these sizes, without launching (a query for
 * tests and benchmarks; no reference counterpart). Writes 8 ints to plan: the register
 * budget (0 heavy: one wave per SIMD; 1 light: two per SIMD; 2 light with non-temporal
 * K/V loads), waves per workgroup, 1 if workgroups take length pairs, query heads per
 * wave, the grid's x, y, z, and the dynamic LDS bytes per workgroup.
 */
int ts_decode_plan(int B, int Hq, int Hkv, int D, int block_size, int max_blocks, int splits,
                   int head_tile, int dtype, int* plan);

/*
 * No counterpart in the reference. For callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): the
 * split-K decode of ts_decode_split + ts_decode_combine, with the fp32 split partials in
 * a static device array of TS_NOALLOC_SCRATCH_BYTES per device instead of caller buffers.
 * The caller passes inputs and `out` as for ts_decode_split (splits == 1 uses no
 * scratch). Returns TS_ETOOBIG, before any launch, when B * Hq * splits * (D + 2) * 4
 * bytes exceed the scratch. Allocates nothing (no hipMalloc, no library allocation); the
 * first call on a device looks up that device's copy of the array, so call it with the
 * stream's device current. Calls on one device share its array: calls that overlap in
 * time on one device (different streams, different threads) race and must be serialised
 * by the caller. Nothing needs clearing between calls: every partial is rewritten.
 */
#define TS_NOALLOC_SCRATCH_BYTES (16 << 20)
int ts_decode_attention_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                const int32_t* block_tables, const int32_t* context_lens,
                                void* out, int B, int Hq, int Hkv, int D, int block_size,
                                int64_t q_stride_b, int64_t q_stride_h, int64_t o_stride_b,
                                int64_t o_stride_h, int64_t k_stride_slot, int64_t k_stride_head,
                                int64_t bt_stride, int max_blocks, int splits, int head_tile,
                                float scale, int dtype, void* stream);

/*
 * The split-K combine pass: out[b, h] = sum_s w_s acc_s / sum_s w_s l_s with
 * w_s = 2^(m_s - max_s m_s); an empty range (m = -inf, l = 0) weighs 0. Head dims up to
 * 256 (TS_EUNSUPPORTED above), any number of splits.
 * Replaces _merge_splits_kernel (triton_attention.py:299-327).
 */
int ts_decode_combine(const float* m, const float* l, const float* acc, void* out, int B,
                      int Hq, int D, int64_t o_stride_b, int64_t o_stride_h, int splits,
                      int dtype, void* stream);

/*
 * Varlen causal prefill attention over the paged cache.
 * Replaces _paged_prefill_kernel as launched by paged_prefill_attention
 * (reference src/tinyserve/triton_prefill.py:50-125, :128-216).
 *
 * Sequence r's queries are rows q_starts[r] .. q_starts[r] + q_lens[r] - 1 of q and
 * are its positions context_lens[r] - q_lens[r] .. context_lens[r] - 1; query at
 * position p attends keys 0 .. p of its own block table. Only those rows of `out`
 * are written. max_q_len (>= every q_lens entry) sizes the grid without a host sync;
 * n_rows, the number of rows of q (0 if unknown), only steers the choice of workgroup
 * shape (mean new tokens per sequence).
 * fp16/bf16 with head_dim 64 or 128 run on MFMA and round the softmax weights to the
 * input dtype before P.V (as the reference kernel does, triton_prefill.py:118); other
 * shapes and fp32 use fp32 FMA throughout.
 */
int ts_prefill_varlen(const void* q, const void* k_cache, const void* v_cache, void* out,
                      const int32_t* block_tables, const int32_t* q_starts,
                      const int32_t* q_lens, const int32_t* context_lens, int R, int Hq,
                      int Hkv, int D, int block_size, int max_q_len, int64_t n_rows,
                      int64_t q_stride_t, int64_t q_stride_h, int64_t o_stride_t,
                      int64_t o_stride_h, int64_t k_stride_slot, int64_t k_stride_head,
                      int64_t bt_stride, float scale, int dtype, void* stream);

/*
 * RMSNorm of every row of x [T, N]:
 *   out = (T)(x * 1/sqrt(mean(x^2) + eps)) * w   (normalise in fp32, multiply in T)
 * Replaces _rms_norm_rows_kernel / rms_norm_rows (triton_fused.py:29-40, :116-126).
 * x, w and out share `dtype`. T == 0 launches nothing.
 */
int ts_rms_norm_rows(const void* x, const void* w, void* out, int T, int N,
                     int64_t x_stride, int64_t o_stride, float eps, int dtype, void* stream);

/*
 * The RoPE tables of T positions (int64): cos / sin [T, D] float32 (row stride `stride`),
 * laid out as cat([angles, angles], -1) with angles[t, i] = positions[t] * theta^(-2i/D)
 * computed in float64. Replaces rope_cos_sin (layers.py:41-65), which the reference's
 * model evaluates with PyTorch ops once per step.
 */
int ts_rope_cos_sin(const int64_t* positions, int T, int D, double theta, float* cos_out,
                    float* sin_out, int64_t stride, void* stream);

/*
 * Per-head RMSNorm + rotate-half RoPE of q and k, and the paged KV-cache write.
 * Replaces _qk_norm_rope_store_kernel / qk_norm_rope_store (triton_fused.py:43-113,
 * :129-177).
 *   q_out[t, h]             = rope(norm(q[t, h]) * q_w)                    (h < Hq)
 *   k_cache[slots[t], kh]   = (cache dtype)(rope(norm(k[t, kh]) * k_w))
 *   v_cache[slots[t], kh]   = (cache dtype)v[t, kh]                         (exact copy)
 * rope(a, b) on the halves: (a cos - b sin, b cos + a sin) with cos/sin [T, D] fp32,
 * of which only columns 0 .. D/2 - 1 are read. q, k, v, weights and q_out share
 * `dtype`; both caches share `cache_dtype`. slots are int64.
 */
int ts_qk_norm_rope_store(const void* q, const void* k, const void* v, void* q_out,
                          const void* q_weight, const void* k_weight, const float* cos,
                          const float* sin, const int64_t* slots, void* k_cache,
                          void* v_cache, int T, int Hq, int Hkv, int D, int64_t q_stride_t,
                          int64_t q_stride_h, int64_t k_stride_t, int64_t k_stride_h,
                          int64_t v_stride_t, int64_t v_stride_h, int64_t o_stride_t,
                          int64_t o_stride_h, int64_t cs_stride_t, int64_t c_stride_slot,
                          int64_t c_stride_head, float eps, int dtype, int cache_dtype,
                          void* stream);

/*
 * Projections of a decode step: out = x . W^T for M rows (a few per sequence) against a
 * weight matrix W [N, K] (row stride w_stride) streamed once. No counterpart in the
 * reference's kernels: these replace the F.linear calls of the decoder layer and the
 * residual adds around them (model.py:137-179) on the decode path; x, W and the outputs
 * share `dtype` (fp16 or bf16). `epilogue`:
 *   TS_ROWS_STORE (0):   out [M, N] (row stride o_stride) = (dtype)(x . W^T)
 *   TS_ROWS_PARTIAL (1): partial [KS][M][N] fp32 = partial sums over KS slices of K, to be
 *                        added by ts_add_rms_norm (KS from ts_rows_gemm_plan; partial
 *                        holds partial_floats floats, at least KS * M * N)
 *   TS_ROWS_SILU (2):    W = [gate; up] (2N rows); out = (dtype)(silu(gate) * up), each
 *                        factor rounded as F.silu / F.linear round it, written
 *                        operand-tiled [Mpad, N] (N % 32 == 0)
 * x_tiled: x is operand-tiled [Mpad, K] (as TS_ROWS_SILU and ts_add_rms_norm write it),
 * else row-major with row stride x_stride. Operand-tiled layout, Mpad = M rounded up to
 * 64: element (m, k) sits at
 *   ((((m/64) * (K/32) + k/32) * 4 + (m%64)/16) * 64 + ((k%32)/8) * 16 + m%16) * 8 + k%8.
 * Pointers 16-byte aligned, strides multiples of 8 elements.
 */
#define TS_ROWS_STORE 0
#define TS_ROWS_PARTIAL 1
#define TS_ROWS_SILU 2
int ts_rows_gemm(const void* x, int x_tiled, int64_t x_stride, const void* w, int64_t w_stride,
                 void* out, int64_t o_stride, float* partial, int64_t partial_floats, int M, int N,
                 int K, int epilogue, int dtype, void* stream);

/*
 * The launch shape ts_rows_gemm picks: out[0] waves per workgroup, out[1] 16-row tiles
 * of W per wave, out[2] 32-column steps per wave, out[3] KS (workgroups along K),
 * out[4] chunks each workgroup walks. No counterpart in the reference.
 */
int ts_rows_gemm_plan(int M, int N, int K, int epilogue, int* out);

/*
 * The residual add + RMSNorm between two projections of a decode step (model.py:170-177:
 * x = x + F.linear(...); h = rms_norm(x)). No counterpart in the reference's kernels.
 *   ks > 0:  x_out = (dtype)(x + partial[0] + ... + partial[ks-1])  (partial [ks][M][N]
 *            fp32 from ts_rows_gemm TS_ROWS_PARTIAL; x_out may be x itself)
 *   ks == 0: the residual is x unchanged (x_out is not written)
 *   h = the RMSNorm of that residual times w, rounded as ts_rms_norm_rows rounds it,
 *       row-major (row stride h_stride) or operand-tiled [Mpad, N] (h_tiled, N % 32 == 0;
 *       padding rows written as zeros).
 * N <= 4096 and a multiple of 8.
 */
int ts_add_rms_norm(const void* x, int64_t x_stride, const float* partial, int ks, const void* w,
                    void* x_out, int64_t xo_stride, void* h, int h_tiled, int64_t h_stride, int M,
                    int N, float eps, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TINYSERVE_AMD_H */
