// Fused per-layer elementwise kernels around attention, for gfx950: hidden-state RMSNorm
// of rows, and the per-head q/k RMSNorm + rotate-half RoPE + paged KV-cache write.
//
// Reference behaviour: src/tinyserve/triton_fused.py:29-113 (kernels) and the numerics
// contract of src/tinyserve/layers.py:14-91: normalise in fp32, round to the input
// dtype, multiply by the weight in the input dtype, rotate in fp32 and round once; the
// cache write is src/tinyserve/kv_cache.py:42-50 (an indexed store with a dtype cast,
// v copied unchanged). Both kernels read every input element once and write every
// output element once.
#include "common.h"

namespace ts {

// W elements at p, as one vector load when ALIGNED (p aligned to W * sizeof(T)).
template <typename T, int W, bool ALIGNED>
struct Chunk {
  T v[W];
  __device__ __forceinline__ void load(const T* p) {
    if constexpr (ALIGNED && W * sizeof(T) >= 4) {
      typedef T VT __attribute__((ext_vector_type(W)));
      const VT x = *reinterpret_cast<const VT*>(p);
#pragma unroll
      for (int i = 0; i < W; ++i) v[i] = x[i];
    } else {
#pragma unroll
      for (int i = 0; i < W; ++i) v[i] = p[i];
    }
  }
  __device__ __forceinline__ void store(T* p) const {
    if constexpr (ALIGNED && W * sizeof(T) >= 4) {
      typedef T VT __attribute__((ext_vector_type(W)));
      VT x;
#pragma unroll
      for (int i = 0; i < W; ++i) x[i] = v[i];
      *reinterpret_cast<VT*>(p) = x;
    } else {
#pragma unroll
      for (int i = 0; i < W; ++i) p[i] = v[i];
    }
  }
};

// ---------------------------------------------------------------------------------
// rms_norm_rows: one wave per row; lane l holds chunks l, l + 64, ... of VEC elements.
// CPL = chunks per lane held in registers (N <= CPL * 64 * VEC).
template <typename T, int CPL, bool ALIGNED>
__global__ __launch_bounds__(256) void rms_norm_rows_kernel(const T* __restrict__ x,
                                                            const T* __restrict__ w,
                                                            T* __restrict__ out, int rows,
                                                            int N, int64_t xs, int64_t os,
                                                            float eps) {
  constexpr int VEC = ALIGNED ? 16 / static_cast<int>(sizeof(T)) : 1;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * xs;
  // The row and the weight are loaded together: the weight's round trip then overlaps
  // the row's instead of following the reduction.
  Chunk<T, VEC, ALIGNED> xv[CPL], wv[CPL];
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int i = (k * 64 + lane) * VEC;
    if (i < N) {
      xv[k].load(xr + i);
      wv[k].load(w + i);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int i = (k * 64 + lane) * VEC;
    if (i < N) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float f = to_f32(xv[k].v[e]);
        ss = fmaf(f, f, ss);
      }
    }
  }
  ss = group_sum<64>(ss);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(N) + eps);
  T* orow = out + row * os;
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    const int i = (k * 64 + lane) * VEC;
    if (i < N) {
      Chunk<T, VEC, ALIGNED> y;
#pragma unroll
      for (int e = 0; e < VEC; ++e) y.v[e] = norm_scale(xv[k].v[e], r, wv[k].v[e]);
      y.store(orow + i);
    }
  }
}

// Rows longer than the register-resident variants: two passes over the row (the
// second read of a row comes from cache, HBM sees one read).
template <typename T>
__global__ __launch_bounds__(256) void rms_norm_rows_long_kernel(const T* __restrict__ x,
                                                                 const T* __restrict__ w,
                                                                 T* __restrict__ out, int rows,
                                                                 int N, int64_t xs, int64_t os,
                                                                 float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * xs;
  float ss = 0.f;
  for (int i = lane; i < N; i += 64) {
    const float f = to_f32(xr[i]);
    ss = fmaf(f, f, ss);
  }
  ss = group_sum<64>(ss);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(N) + eps);
  T* orow = out + row * os;
  for (int i = lane; i < N; i += 64) orow[i] = norm_scale(xr[i], r, w[i]);
}

template <typename T>
static int launch_rms(const void* x, const void* w, void* out, int rows, int N, int64_t xs,
                      int64_t os, float eps, hipStream_t st) {
  constexpr int VEC = 16 / sizeof(T);
  const bool aligned = N % VEC == 0 && xs % VEC == 0 && os % VEC == 0 &&
                       (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                        reinterpret_cast<uintptr_t>(out)) % 16 == 0;
  const T* xp = static_cast<const T*>(x);
  const T* wp = static_cast<const T*>(w);
  T* op = static_cast<T*>(out);
  // Fewer rows than four per CU (a decode step's batch): one wave per workgroup, so the
  // rows spread over as many CUs; otherwise four waves (rows) per workgroup.
  const int wpb = rows < 4 * compute_units() ? 1 : 4;
  dim3 grid((rows + wpb - 1) / wpb), block(64 * wpb);
  const int per_chunk = 64 * (aligned ? VEC : 1);
  const int cpl = (N + per_chunk - 1) / per_chunk;
#define TS_RMS(C, A) \
  hipLaunchKernelGGL((rms_norm_rows_kernel<T, C, A>), grid, block, 0, st, xp, wp, op, rows, N, xs, os, eps)
  if (aligned) {
    if (cpl <= 1) TS_RMS(1, true);
    else if (cpl <= 2) TS_RMS(2, true);
    else if (cpl <= 4) TS_RMS(4, true);
    else if (cpl <= 8) TS_RMS(8, true);
    else hipLaunchKernelGGL(rms_norm_rows_long_kernel<T>, grid, block, 0, st, xp, wp, op, rows, N, xs, os, eps);
  } else {
    if (cpl <= 1) TS_RMS(1, false);
    else if (cpl <= 4) TS_RMS(4, false);
    else hipLaunchKernelGGL(rms_norm_rows_long_kernel<T>, grid, block, 0, st, xp, wp, op, rows, N, xs, os, eps);
  }
#undef TS_RMS
  return launch_status();
}

// ---------------------------------------------------------------------------------
// qk_norm_rope_store: LPH lanes per head vector; lane j holds elements
// j*W .. j*W+W-1 of the first half and the same of the second half, so every rotate-half
// pair (i, i + D/2) is in one lane. Units per token, in order: Hq query heads (to
// q_out), Hkv key heads (to k_cache), Hkv value heads (to v_cache).
struct QkArgs {
  const void* q;
  const void* k;
  const void* v;
  void* q_out;
  const void* qw;
  const void* kw;
  const float* cos;
  const float* sin;
  const int64_t* slots;
  void* kc;
  void* vc;
  int T;
  int Hq;
  int Hkv;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh, cs_st, c_ss, c_sh;
  float eps;
};

template <typename T, typename TC, int D, bool ALIGNED>
__global__ __launch_bounds__(256) void qk_norm_rope_store_kernel(const QkArgs a) {
#pragma clang fp contract(off)
  constexpr int HALF = D / 2;
  constexpr int WMAX = 16 / static_cast<int>(sizeof(T));
  constexpr int W = HALF < WMAX ? HALF : WMAX;
  constexpr int LPH = HALF / W;
  static_assert(LPH >= 1 && LPH <= 64 && (LPH & (LPH - 1)) == 0, "lanes per head");
  const int units = a.Hq + 2 * a.Hkv;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t unit = gid / LPH;
  const int j = static_cast<int>(gid % LPH);
  if (unit >= static_cast<int64_t>(a.T) * units) return;
  const int t = static_cast<int>(unit / units);
  const int u = static_cast<int>(unit % units);
  const int off = j * W;

  if (u >= a.Hq + a.Hkv) {  // value head: an exact copy (cast) into the cache
    const int kh = u - a.Hq - a.Hkv;
    const T* src = static_cast<const T*>(a.v) + t * a.v_st + kh * a.v_sh;
    TC* dst = static_cast<TC*>(a.vc) + a.slots[t] * a.c_ss + kh * a.c_sh;
    Chunk<T, W, ALIGNED> x0, x1;
    x0.load(src + off);
    x1.load(src + HALF + off);
    Chunk<TC, W, ALIGNED> y0, y1;
#pragma unroll
    for (int e = 0; e < W; ++e) {
      y0.v[e] = from_f32<TC>(to_f32(x0.v[e]));
      y1.v[e] = from_f32<TC>(to_f32(x1.v[e]));
    }
    y0.store(dst + off);
    y1.store(dst + HALF + off);
    return;
  }

  const bool is_q = u < a.Hq;
  const int hh = is_q ? u : u - a.Hq;
  const T* src = is_q ? static_cast<const T*>(a.q) + t * a.q_st + hh * a.q_sh
                      : static_cast<const T*>(a.k) + t * a.k_st + hh * a.k_sh;
  const T* wp = static_cast<const T*>(is_q ? a.qw : a.kw);
  Chunk<T, W, ALIGNED> xa, xb, wa, wb;
  xa.load(src + off);
  xb.load(src + HALF + off);
  wa.load(wp + off);
  wb.load(wp + HALF + off);
  // The angles and the key's slot are loaded with the head, not after the reduction.
  float c[W], s[W];
#pragma unroll
  for (int e = 0; e < W; ++e) {
    c[e] = a.cos[t * a.cs_st + off + e];
    s[e] = a.sin[t * a.cs_st + off + e];
  }
  const int64_t slot = is_q ? 0 : a.slots[t];
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < W; ++e) {
    const float fa = to_f32(xa.v[e]), fb = to_f32(xb.v[e]);
    ss += fa * fa;
    ss += fb * fb;
  }
  ss = group_sum<LPH>(ss);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(D) + a.eps);
  Chunk<T, W, ALIGNED> ya, yb;
#pragma unroll
  for (int e = 0; e < W; ++e) {
    const float na = to_f32(norm_scale(xa.v[e], r, wa.v[e]));
    const float nb = to_f32(norm_scale(xb.v[e], r, wb.v[e]));
    const float ra = na * c[e] - nb * s[e];
    const float rb = nb * c[e] + na * s[e];
    ya.v[e] = from_f32<T>(ra);
    yb.v[e] = from_f32<T>(rb);
  }
  if (is_q) {
    T* dst = static_cast<T*>(a.q_out) + t * a.o_st + hh * a.o_sh;
    ya.store(dst + off);
    yb.store(dst + HALF + off);
  } else {
    TC* dst = static_cast<TC*>(a.kc) + slot * a.c_ss + hh * a.c_sh;
    Chunk<TC, W, ALIGNED> za, zb;
#pragma unroll
    for (int e = 0; e < W; ++e) {
      za.v[e] = from_f32<TC>(to_f32(ya.v[e]));
      zb.v[e] = from_f32<TC>(to_f32(yb.v[e]));
    }
    za.store(dst + off);
    zb.store(dst + HALF + off);
  }
}

template <typename T, typename TC, int D>
static int launch_qk_d(const QkArgs& a, hipStream_t st) {
  constexpr int HALF = D / 2;
  constexpr int WMAX = 16 / static_cast<int>(sizeof(T));
  constexpr int W = HALF < WMAX ? HALF : WMAX;
  constexpr int LPH = HALF / W;
  // Vector loads need every row start aligned to W elements of both T and TC.
  const int64_t strides[] = {a.q_st, a.q_sh, a.k_st, a.k_sh, a.v_st, a.v_sh,
                             a.o_st, a.o_sh, a.c_ss, a.c_sh};
  bool aligned = true;
  for (int64_t s : strides) aligned &= (s % W) == 0;
  const uintptr_t pt = reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.k) |
                       reinterpret_cast<uintptr_t>(a.v) | reinterpret_cast<uintptr_t>(a.q_out) |
                       reinterpret_cast<uintptr_t>(a.qw) | reinterpret_cast<uintptr_t>(a.kw);
  const uintptr_t pc = reinterpret_cast<uintptr_t>(a.kc) | reinterpret_cast<uintptr_t>(a.vc);
  aligned &= pt % (W * sizeof(T)) == 0 && pc % (W * sizeof(TC)) == 0;
  const int64_t threads = static_cast<int64_t>(a.T) * (a.Hq + 2 * a.Hkv) * LPH;
  // Few tokens (a decode step): one-wave workgroups, spread over more CUs.
  const int bt = threads < 256 * static_cast<int64_t>(compute_units()) ? 64 : 256;
  dim3 grid(static_cast<unsigned>((threads + bt - 1) / bt)), block(bt);
  if (aligned)
    hipLaunchKernelGGL((qk_norm_rope_store_kernel<T, TC, D, true>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((qk_norm_rope_store_kernel<T, TC, D, false>), grid, block, 0, st, a);
  return launch_status();
}

template <typename T, typename TC>
static int launch_qk(const QkArgs& a, int D, hipStream_t st) {
  switch (D) {
    case 8: return launch_qk_d<T, TC, 8>(a, st);
    case 16: return launch_qk_d<T, TC, 16>(a, st);
    case 32: return launch_qk_d<T, TC, 32>(a, st);
    case 64: return launch_qk_d<T, TC, 64>(a, st);
    case 128: return launch_qk_d<T, TC, 128>(a, st);
    case 256: return launch_qk_d<T, TC, 256>(a, st);
    default: return TS_EUNSUPPORTED;
  }
}

template <typename T>
static int launch_qk_cache(const QkArgs& a, int D, int cache_dtype, hipStream_t st) {
  switch (cache_dtype) {
    case TS_F32: return launch_qk<T, float>(a, D, st);
    case TS_F16: return launch_qk<T, f16>(a, D, st);
    case TS_BF16: return launch_qk<T, bf16>(a, D, st);
    default: return TS_EUNSUPPORTED;
  }
}

// ---------------------------------------------------------------------------------
// rope_cos_sin: the rotation tables of layers.py:41-65 for T positions, one thread per
// (position, pair i): inv_freq = theta^(-2i / D) and the angle p * inv_freq in float64,
// cos / sin in float64 rounded once to float32, written to columns i and i + D/2.
__global__ __launch_bounds__(256) void rope_cos_sin_kernel(const int64_t* __restrict__ pos, int T, int D,
                                                           double theta, float* __restrict__ cos_out,
                                                           float* __restrict__ sin_out, int64_t stride) {
  const int half = D / 2;
  const int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (u >= static_cast<int64_t>(T) * half) return;
  const int t = static_cast<int>(u / half), i = static_cast<int>(u % half);
  const double inv_freq = pow(theta, -static_cast<double>(2 * i) / static_cast<double>(D));
  const double ang = static_cast<double>(pos[t]) * inv_freq;
  const float c = static_cast<float>(cos(ang)), sn = static_cast<float>(sin(ang));
  cos_out[t * stride + i] = c;
  cos_out[t * stride + i + half] = c;
  sin_out[t * stride + i] = sn;
  sin_out[t * stride + i + half] = sn;
}

}  // namespace ts

using namespace ts;

extern "C" int ts_rope_cos_sin(const int64_t* positions, int T, int D, double theta, float* cos_out,
                               float* sin_out, int64_t stride, void* stream) {
  if (T < 0 || D < 2 || D % 2 || stride < D || !(theta > 0.0)) return TS_EINVAL;
  if (T == 0) return 0;
  if (!positions || !cos_out || !sin_out) return TS_EINVAL;
  const int64_t n = static_cast<int64_t>(T) * (D / 2);
  hipLaunchKernelGGL(rope_cos_sin_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), positions, T, D, theta, cos_out, sin_out, stride);
  return launch_status();
}

extern "C" int ts_rms_norm_rows(const void* x, const void* w, void* out, int T, int N,
                                int64_t x_stride, int64_t o_stride, float eps, int dtype,
                                void* stream) {
  if (T < 0 || N <= 0) return TS_EINVAL;
  if (T == 0) return 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TS_F32: return launch_rms<float>(x, w, out, T, N, x_stride, o_stride, eps, st);
    case TS_F16: return launch_rms<f16>(x, w, out, T, N, x_stride, o_stride, eps, st);
    case TS_BF16: return launch_rms<bf16>(x, w, out, T, N, x_stride, o_stride, eps, st);
    default: return TS_EUNSUPPORTED;
  }
}

extern "C" int ts_qk_norm_rope_store(
    const void* q, const void* k, const void* v, void* q_out, const void* q_weight,
    const void* k_weight, const float* cos, const float* sin, const int64_t* slots,
    void* k_cache, void* v_cache, int T, int Hq, int Hkv, int D, int64_t q_stride_t,
    int64_t q_stride_h, int64_t k_stride_t, int64_t k_stride_h, int64_t v_stride_t,
    int64_t v_stride_h, int64_t o_stride_t, int64_t o_stride_h, int64_t cs_stride_t,
    int64_t c_stride_slot, int64_t c_stride_head, float eps, int dtype, int cache_dtype,
    void* stream) {
  if (T < 0 || Hq <= 0 || Hkv <= 0 || D < 2 || D % 2 || !is_pow2(D / 2)) return TS_EINVAL;
  if (T == 0) return 0;
  QkArgs a{q, k, v, q_out, q_weight, k_weight, cos, sin, slots, k_cache, v_cache, T, Hq, Hkv,
           q_stride_t, q_stride_h, k_stride_t, k_stride_h, v_stride_t, v_stride_h,
           o_stride_t, o_stride_h, cs_stride_t, c_stride_slot, c_stride_head, eps};
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case TS_F32: return launch_qk_cache<float>(a, D, cache_dtype, st);
    case TS_F16: return launch_qk_cache<f16>(a, D, cache_dtype, st);
    case TS_BF16: return launch_qk_cache<bf16>(a, D, cache_dtype, st);
    default: return TS_EUNSUPPORTED;
  }
}
