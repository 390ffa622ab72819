// N-first normalisation kernels: LayerNorm with per-model affine, and
// eval-mode BatchNorm per (model, channel).  Both are HBM-bound: one read and
// one write of the activation, statistics in fp32 registers (LayerNorm rows
// longer than one wave holds are read three times by one workgroup each).
#include "wc_common.h"

namespace wc {
namespace {

constexpr int kNormBlock = 256;

template <typename T, int V> struct LoadV;
template <typename T> struct LoadV<T, 1> {
  static __device__ __forceinline__ void ld(const T* p, float* o) { o[0] = to_f32(p[0]); }
  static __device__ __forceinline__ void st(T* p, const float* o) { p[0] = from_f32<T>(o[0]); }
};
template <> struct LoadV<float, 4> {
  static __device__ __forceinline__ void ld(const float* p, float* o) {
    const float4 v = *reinterpret_cast<const float4*>(p);
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
  }
  static __device__ __forceinline__ void st(float* p, const float* o) {
    *reinterpret_cast<float4*>(p) = make_float4(o[0], o[1], o[2], o[3]);
  }
};
template <typename H> struct LoadV8x16 {
  static __device__ __forceinline__ void ld(const H* p, float* o) {
    typedef H h8 __attribute__((ext_vector_type(8)));
    const h8 v = *reinterpret_cast<const h8*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = static_cast<float>(v[i]);
  }
  static __device__ __forceinline__ void st(H* p, const float* o) {
    typedef H h8 __attribute__((ext_vector_type(8)));
    h8 v;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = static_cast<H>(o[i]);
    *reinterpret_cast<h8*>(p) = v;
  }
};
template <> struct LoadV<bf16, 8> : LoadV8x16<bf16> {};
template <> struct LoadV<f16, 8> : LoadV8x16<f16> {};

__device__ __forceinline__ float lanes_sum(float v, int lanes) {
  for (int off = lanes >> 1; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// One group of `lanes` adjacent lanes per row; lane j of the group owns the
// V-element vectors at (it * lanes + j) * V for it < ITEMS.
template <typename T, typename P, int V, int ITEMS>
__global__ __launch_bounds__(kNormBlock) void layernorm_kernel(
    const T* __restrict__ x, int64_t xms, int64_t xrs, const P* __restrict__ gamma,
    const P* __restrict__ beta, T* __restrict__ y, int64_t yms, int64_t yrs, uint32_t rows_total,
    FastDiv rows_per_model, int dim, int lanes_log2, float eps) {
  const int lanes = 1 << lanes_log2;
  const int tid = threadIdx.x;
  const int j = tid & (lanes - 1);
  const uint32_t row = blockIdx.x * (kNormBlock >> lanes_log2) + (tid >> lanes_log2);
  if (row >= rows_total) return;  // whole lane groups leave together
  const uint32_t m = fdiv(row, rows_per_model);
  const uint32_t r = row - m * rows_per_model.d;
  const T* xr = x + static_cast<int64_t>(m) * xms + static_cast<int64_t>(r) * xrs;
  T* yr = y + static_cast<int64_t>(m) * yms + static_cast<int64_t>(r) * yrs;
  const P* g = gamma + static_cast<int64_t>(m) * dim;
  const P* b = beta ? beta + static_cast<int64_t>(m) * dim : nullptr;

  float v[ITEMS][V];
  float s = 0.f;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int e = (it * lanes + j) * V;
    if (e < dim) {
      LoadV<T, V>::ld(xr + e, v[it]);
#pragma unroll
      for (int q = 0; q < V; ++q) s += v[it][q];
    }
  }
  const float mean = lanes_sum(s, lanes) / static_cast<float>(dim);
  float s2 = 0.f;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int e = (it * lanes + j) * V;
    if (e < dim) {
#pragma unroll
      for (int q = 0; q < V; ++q) {
        const float d = v[it][q] - mean;
        s2 += d * d;
      }
    }
  }
  const float var = lanes_sum(s2, lanes) / static_cast<float>(dim);
  const float denom = sqrtf(var + eps);
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int e = (it * lanes + j) * V;
    if (e < dim) {
      float o[V];
#pragma unroll
      for (int q = 0; q < V; ++q) {
        const float bq = b ? to_f32(b[e + q]) : 0.f;
        o[q] = ((v[it][q] - mean) / denom) * to_f32(g[e + q]) + bq;
      }
      LoadV<T, V>::st(yr + e, o);
    }
  }
}

// Sum of `v` over the 256 threads of the workgroup (red: 4 floats of LDS).
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = lanes_sum(v, 64);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  const float s = red[0] + red[1] + red[2] + red[3];
  __syncthreads();                                   // red is reused by the next reduction
  return s;
}

// Rows longer than one wave can hold in registers: one workgroup per row (grid-stride over
// rows), three passes over the row (mean, variance about the mean, normalise), fp32 statistics
// and the same expression as layernorm_kernel.
template <typename T, typename P, int V>
__global__ __launch_bounds__(kNormBlock) void layernorm_rows_kernel(
    const T* __restrict__ x, int64_t xms, int64_t xrs, const P* __restrict__ gamma,
    const P* __restrict__ beta, T* __restrict__ y, int64_t yms, int64_t yrs, uint32_t rows_total,
    FastDiv rows_per_model, int dim, float eps) {
  static_assert(kNormBlock == 256, "block_sum assumes 4 waves");
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const int nv = dim / V;                            // V divides dim
  for (uint32_t row = blockIdx.x; row < rows_total; row += gridDim.x) {
    const uint32_t m = fdiv(row, rows_per_model);
    const uint32_t r = row - m * rows_per_model.d;
    const T* xr = x + static_cast<int64_t>(m) * xms + static_cast<int64_t>(r) * xrs;
    T* yr = y + static_cast<int64_t>(m) * yms + static_cast<int64_t>(r) * yrs;
    const P* g = gamma + static_cast<int64_t>(m) * dim;
    const P* b = beta ? beta + static_cast<int64_t>(m) * dim : nullptr;
    float s = 0.f;
    for (int i = tid; i < nv; i += kNormBlock) {
      float v[V];
      LoadV<T, V>::ld(xr + static_cast<int64_t>(i) * V, v);
#pragma unroll
      for (int q = 0; q < V; ++q) s += v[q];
    }
    const float mean = block_sum(s, red) / static_cast<float>(dim);
    float s2 = 0.f;
    for (int i = tid; i < nv; i += kNormBlock) {
      float v[V];
      LoadV<T, V>::ld(xr + static_cast<int64_t>(i) * V, v);
#pragma unroll
      for (int q = 0; q < V; ++q) {
        const float d = v[q] - mean;
        s2 += d * d;
      }
    }
    const float var = block_sum(s2, red) / static_cast<float>(dim);
    const float denom = sqrtf(var + eps);
    for (int i = tid; i < nv; i += kNormBlock) {
      const int64_t e = static_cast<int64_t>(i) * V;
      float v[V], o[V];
      LoadV<T, V>::ld(xr + e, v);
#pragma unroll
      for (int q = 0; q < V; ++q) {
        const float bq = b ? to_f32(b[e + q]) : 0.f;
        o[q] = ((v[q] - mean) / denom) * to_f32(g[e + q]) + bq;
      }
      LoadV<T, V>::st(yr + e, o);
    }
  }
}

// eval BatchNorm: one 16-byte (or narrower) vector per thread per unroll slot
template <typename T, typename P, int V>
__global__ __launch_bounds__(kNormBlock) void bn_eval_kernel(
    const T* __restrict__ x, int64_t xsn, int64_t xsb, const P* __restrict__ w,
    const P* __restrict__ bias, const P* __restrict__ rm, const P* __restrict__ rv, float eps,
    T* __restrict__ y, uint32_t total_chunks, FastDiv cpp, FastDiv nch, FastDiv nb, int hw,
    int relu) {
  const uint32_t k = blockIdx.x * kNormBlock + threadIdx.x;
  if (k >= total_chunks) return;
  const uint32_t p = fdiv(k, cpp);            // plane = (i * B + b) * C + ch
  const uint32_t c = k - p * cpp.d;
  const uint32_t ib = fdiv(p, nch);
  const uint32_t ch = p - ib * nch.d;
  const uint32_t i = fdiv(ib, nb);
  const uint32_t bb = ib - i * nb.d;
  const uint32_t pi = i * nch.d + ch;          // parameter index (model, channel)
  const float invstd = 1.0f / sqrtf(to_f32(rv[pi]) + eps);
  const float alpha = w ? invstd * to_f32(w[pi]) : invstd;
  const float beta = (bias ? to_f32(bias[pi]) : 0.f) - to_f32(rm[pi]) * alpha;
  const int64_t e = static_cast<int64_t>(c) * V;
  const T* xp = x + static_cast<int64_t>(i) * xsn + static_cast<int64_t>(bb) * xsb +
                static_cast<int64_t>(ch) * hw + e;
  T* yp = y + static_cast<int64_t>(p) * hw + e;
  float v[V];
  LoadV<T, V>::ld(xp, v);
#pragma unroll
  for (int q = 0; q < V; ++q) {
    float o = v[q] * alpha + beta;
    if (relu) o = o > 0.f ? o : 0.f;
    v[q] = o;
  }
  LoadV<T, V>::st(yp, v);
}

// DPP lane permutation inside a 16-lane row (register-to-register)
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF,
                                                               0xF, true));
}

// Sum over groups of L adjacent lanes (L a power of two <= 64), delivered to
// every lane of the group: DPP inside 16-lane rows, lane exchange beyond.
template <int L>
__device__ __forceinline__ float group_reduce(float v) {
  if (L >= 2) v += dpp_f<0xB1>(v);    // quad_perm [1,0,3,2]
  if (L >= 4) v += dpp_f<0x4E>(v);    // quad_perm [2,3,0,1]
  if (L >= 8) v += dpp_f<0x141>(v);   // row_half_mirror
  if (L >= 16) v += dpp_f<0x140>(v);  // row_mirror
  if (L >= 32) v += __shfl_xor(v, 16, 64);
  if (L >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

// Vector LayerNorm: a group of L lanes owns RPG consecutive rows of one model
// (rows_per_model % RPG == 0); lane j holds the 16-byte vectors (it * L + j)
// of each row.  All RPG x ITEMS row loads are issued before any arithmetic, so
// a wave keeps RPG x ITEMS x 1 KB in flight; gamma / beta are read once per
// group as 16-byte vectors; two-pass statistics in fp32 registers; one
// reciprocal square root per row.
// The embedding gather in front of the LayerNorm (GATHER): row r of model m reads table row
// ids[r] (shared ids) or ids[m * rows + r] of model m (x = the table, xms its model stride); an
// id outside [0, vocab) reads a zero row, as the gather kernel writes one, and sets *err.
struct LnGather {
  const int64_t* ids;
  int64_t vocab;
  int ids_shared;
  int32_t* err;
};

template <typename T, typename P, int L, int ITEMS, int RPG, bool GATHER = false>
__global__ __launch_bounds__(kNormBlock) void layernorm_vec_kernel(
    const T* __restrict__ x, int64_t xms, int64_t xrs, const P* __restrict__ gamma,
    const P* __restrict__ beta, T* __restrict__ y, int64_t yms, int64_t yrs, uint32_t rows_total,
    FastDiv rows_per_model, int dim, float eps, LnGather gth) {
  constexpr int V = 16 / sizeof(T);
  const int tid = threadIdx.x;
  const int j = tid & (L - 1);
  const uint32_t row0 = (blockIdx.x * (kNormBlock / L) + tid / L) * RPG;
  if (row0 >= rows_total) return;  // whole lane groups leave together
  const uint32_t m = fdiv(row0, rows_per_model);
  const uint32_t r0 = row0 - m * rows_per_model.d;
  const T* xr = x + static_cast<int64_t>(m) * xms + static_cast<int64_t>(r0) * xrs;
  T* yr = y + static_cast<int64_t>(m) * yms + static_cast<int64_t>(r0) * yrs;

  float v[RPG][ITEMS][V];
#pragma unroll
  for (int r = 0; r < RPG; ++r) {
    const T* src = xr + static_cast<int64_t>(r) * xrs;
    bool ok = true;
    if constexpr (GATHER) {
      const int64_t id = gth.ids[gth.ids_shared ? static_cast<int64_t>(r0 + r)
                                                : static_cast<int64_t>(m) * rows_per_model.d + r0 + r];
      ok = id >= 0 && id < gth.vocab;
      src = x + static_cast<int64_t>(m) * xms + (ok ? id : 0) * dim;
      if (!ok && j == 0 && gth.err) *gth.err = 1;
    }
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
      const int e = (it * L + j) * V;
      if (e < dim) {
        if (ok) {
          LoadV<T, V>::ld(src + e, v[r][it]);
        } else {
#pragma unroll
          for (int q = 0; q < V; ++q) v[r][it][q] = 0.f;
        }
      }
    }
  }
  float gv[ITEMS][V], bv[ITEMS][V];
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int e = (it * L + j) * V;
    if (e < dim) {
      const P* g = gamma + static_cast<int64_t>(m) * dim + e;
      const P* b = beta ? beta + static_cast<int64_t>(m) * dim + e : nullptr;
#pragma unroll
      for (int q = 0; q < V; q += 16 / sizeof(P)) {
        LoadV<P, 16 / sizeof(P)>::ld(g + q, &gv[it][q]);
        if (b) LoadV<P, 16 / sizeof(P)>::ld(b + q, &bv[it][q]);
        else
#pragma unroll
          for (int u = 0; u < static_cast<int>(16 / sizeof(P)); ++u) bv[it][q + u] = 0.f;
      }
    }
  }
  const float inv_d = 1.0f / static_cast<float>(dim);
#pragma unroll
  for (int r = 0; r < RPG; ++r) {
    float s = 0.f;
#pragma unroll
    for (int it = 0; it < ITEMS; ++it)
      if ((it * L + j) * V < dim)
#pragma unroll
        for (int q = 0; q < V; ++q) s += v[r][it][q];
    const float mean = group_reduce<L>(s) * inv_d;
    float s2 = 0.f;
#pragma unroll
    for (int it = 0; it < ITEMS; ++it)
      if ((it * L + j) * V < dim)
#pragma unroll
        for (int q = 0; q < V; ++q) {
          const float d = v[r][it][q] - mean;
          s2 += d * d;
        }
    const float rstd = 1.0f / sqrtf(group_reduce<L>(s2) * inv_d + eps);
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
      const int e = (it * L + j) * V;
      if (e < dim) {
        float o[V];
#pragma unroll
        for (int q = 0; q < V; ++q) o[q] = (v[r][it][q] - mean) * rstd * gv[it][q] + bv[it][q];
        LoadV<T, V>::st(yr + static_cast<int64_t>(r) * yrs + e, o);
      }
    }
  }
}

template <typename T, typename P, int V>
int32_t launch_layernorm_v(const T* x, int64_t xms, int64_t xrs, const P* g, const P* b, T* y,
                           int64_t yms, int64_t yrs, int64_t n, int64_t rpm, int dim, float eps,
                           hipStream_t st) {
  const int64_t nvec = cdiv(dim, V);
  int lanes_log2 = 0;
  while ((1 << lanes_log2) < nvec && lanes_log2 < 6) ++lanes_log2;
  const int lanes = 1 << lanes_log2;
  const int items = static_cast<int>(cdiv(nvec, lanes));
  const uint32_t rows_total = static_cast<uint32_t>(n * rpm);
  const int rows_per_block = kNormBlock >> lanes_log2;
  const dim3 grid(static_cast<uint32_t>(cdiv(rows_total, rows_per_block)));
  const FastDiv fr = make_fastdiv(static_cast<uint32_t>(rpm));
#define WC_LN_CASE(IT)                                                                        \
  if (items <= IT) {                                                                          \
    layernorm_kernel<T, P, V, IT><<<grid, kNormBlock, 0, st>>>(x, xms, xrs, g, b, y, yms, yrs, \
                                                               rows_total, fr, dim, lanes_log2, eps); \
    return check_launch("wc_layernorm");                                                      \
  }
  WC_LN_CASE(1)
  WC_LN_CASE(2)
  WC_LN_CASE(4)
  WC_LN_CASE(8)
  WC_LN_CASE(16)
#undef WC_LN_CASE
  return set_error(WC_ERR_LIMIT, "wc_layernorm: dim %d too large", dim);
}

template <typename T, typename P>
int32_t launch_layernorm(const void* x, int64_t xms, int64_t xrs, const void* g, const void* b,
                         void* y, int64_t yms, int64_t yrs, int64_t n, int64_t rpm, int64_t dim,
                         float eps, hipStream_t st) {
  constexpr int VMAX = 16 / sizeof(T);
  const int es = sizeof(T);
  const int vb = common_vec_bytes({reinterpret_cast<uintptr_t>(x), reinterpret_cast<uintptr_t>(y),
                                   reinterpret_cast<uintptr_t>(g), reinterpret_cast<uintptr_t>(b),
                                   ubytes(dim, es),
                                   ubytes(xms, es), ubytes(xrs, es),
                                   ubytes(yms, es), ubytes(yrs, es),
                                   static_cast<uint64_t>(dim * sizeof(P))});
  const bool vec_ok = vb >= 16;
  if (vec_ok && dim % VMAX == 0 && dim <= 4 * 64 * VMAX) {
    const int64_t nvec = dim / VMAX;
    const uint32_t rows_total = static_cast<uint32_t>(n * rpm);
    const FastDiv fr = make_fastdiv(static_cast<uint32_t>(rpm));
    const int rpg = (rpm % 4 == 0) ? 4 : ((rpm % 2 == 0) ? 2 : 1);
    const T* xt = static_cast<const T*>(x);
    const P* gt = static_cast<const P*>(g);
    const P* bt = static_cast<const P*>(b);
    T* yt = static_cast<T*>(y);
#define WC_LNV(L, IT, R)                                                                                 \
  if (nvec <= (L) * (IT) && rpg == (R)) {                                                              \
    const int64_t groups = cdiv(rows_total, R);                                                       \
    const dim3 grid(static_cast<uint32_t>(cdiv(groups, kNormBlock / (L))));                          \
    layernorm_vec_kernel<T, P, L, IT, R><<<grid, kNormBlock, 0, st>>>(xt, xms, xrs, gt, bt, yt, yms, yrs, \
                                                                      rows_total, fr, (int)dim, eps,   \
                                                                      LnGather{});                    \
    return check_launch("wc_layernorm");                                                              \
  }
#define WC_LNV_R(L, IT) WC_LNV(L, IT, 4) WC_LNV(L, IT, 2) WC_LNV(L, IT, 1)
    WC_LNV_R(4, 1) WC_LNV_R(8, 1) WC_LNV_R(16, 1) WC_LNV_R(32, 1) WC_LNV_R(64, 1)
    WC_LNV_R(64, 2) WC_LNV_R(64, 4)
#undef WC_LNV_R
#undef WC_LNV
  }
  if (vec_ok && dim <= 16 * 64 * VMAX)
    return launch_layernorm_v<T, P, VMAX>(static_cast<const T*>(x), xms, xrs,
                                          static_cast<const P*>(g), static_cast<const P*>(b),
                                          static_cast<T*>(y), yms, yrs, n, rpm, (int)dim, eps, st);
  if (!vec_ok && dim <= 16 * 64)
    return launch_layernorm_v<T, P, 1>(static_cast<const T*>(x), xms, xrs, static_cast<const P*>(g),
                                       static_cast<const P*>(b), static_cast<T*>(y), yms, yrs, n, rpm,
                                       (int)dim, eps, st);
  // longer rows: one workgroup per row (vec_ok implies VMAX divides dim)
  const uint32_t rows_total = static_cast<uint32_t>(n * rpm);
  const FastDiv fr = make_fastdiv(static_cast<uint32_t>(rpm));
  const dim3 grid(rows_total < 65536u ? rows_total : 65536u);
  if (vec_ok)
    layernorm_rows_kernel<T, P, VMAX><<<grid, kNormBlock, 0, st>>>(
        static_cast<const T*>(x), xms, xrs, static_cast<const P*>(g), static_cast<const P*>(b),
        static_cast<T*>(y), yms, yrs, rows_total, fr, (int)dim, eps);
  else
    layernorm_rows_kernel<T, P, 1><<<grid, kNormBlock, 0, st>>>(
        static_cast<const T*>(x), xms, xrs, static_cast<const P*>(g), static_cast<const P*>(b),
        static_cast<T*>(y), yms, yrs, rows_total, fr, (int)dim, eps);
  return check_launch("wc_layernorm");
}

// Embedding gather + LayerNorm in one pass: the vector-path LayerNorm kernel reading its rows
// through the ids, with the shape selection of launch_layernorm's vector path, so the output
// equals wc_embedding_gather followed by wc_layernorm bit for bit.  WC_ERR_LIMIT (nothing
// launched) where that path does not apply.
template <typename T, typename P>
int32_t launch_emb_layernorm(const void* w, int64_t n, int64_t vocab, int64_t dim, const int64_t* ids,
                             int64_t rows, int ids_shared, const void* g, const void* b, float eps, void* y,
                             int32_t* err, hipStream_t st) {
  constexpr int VMAX = 16 / sizeof(T);
  const int es = sizeof(T);
  const int vb = common_vec_bytes({reinterpret_cast<uintptr_t>(w), reinterpret_cast<uintptr_t>(y),
                                   reinterpret_cast<uintptr_t>(g), reinterpret_cast<uintptr_t>(b),
                                   ubytes(dim, es), static_cast<uint64_t>(dim * sizeof(P))});
  if (!(vb >= 16 && dim % VMAX == 0 && dim <= 4 * 64 * VMAX))
    return set_error(WC_ERR_LIMIT, "wc_embedding_layernorm: dim %lld or alignment outside the fused kernel "
                     "(16-byte rows, dim a multiple of %d up to %d)", static_cast<long long>(dim), VMAX,
                     4 * 64 * VMAX);
  const int64_t nvec = dim / VMAX;
  const uint32_t rows_total = static_cast<uint32_t>(n * rows);
  const FastDiv fr = make_fastdiv(static_cast<uint32_t>(rows));
  const int rpg = (rows % 4 == 0) ? 4 : ((rows % 2 == 0) ? 2 : 1);
  const T* wt = static_cast<const T*>(w);
  const P* gt = static_cast<const P*>(g);
  const P* bt = static_cast<const P*>(b);
  T* yt = static_cast<T*>(y);
  const LnGather gth{ids, vocab, ids_shared, err};
#define WC_ELN(L, IT, R)                                                                                \
  if (nvec <= (L) * (IT) && rpg == (R)) {                                                             \
    const int64_t groups = cdiv(rows_total, R);                                                      \
    const dim3 grid(static_cast<uint32_t>(cdiv(groups, kNormBlock / (L))));                         \
    layernorm_vec_kernel<T, P, L, IT, R, true><<<grid, kNormBlock, 0, st>>>(                         \
        wt, vocab * dim, 0, gt, bt, yt, rows * dim, dim, rows_total, fr, (int)dim, eps, gth);       \
    return check_launch("wc_embedding_layernorm");                                                  \
  }
#define WC_ELN_R(L, IT) WC_ELN(L, IT, 4) WC_ELN(L, IT, 2) WC_ELN(L, IT, 1)
  WC_ELN_R(4, 1) WC_ELN_R(8, 1) WC_ELN_R(16, 1) WC_ELN_R(32, 1) WC_ELN_R(64, 1)
  WC_ELN_R(64, 2) WC_ELN_R(64, 4)
#undef WC_ELN_R
#undef WC_ELN
  return set_error(WC_ERR_LIMIT, "wc_embedding_layernorm: dim %lld too large", static_cast<long long>(dim));
}

template <typename T, typename P>
int32_t launch_bn(const void* x, int64_t xsn, int64_t xsb, const void* w, const void* bias,
                  const void* rm, const void* rv, float eps, void* y, int64_t n, int64_t b,
                  int64_t c, int64_t hw, int act, hipStream_t st) {
  constexpr int VMAX = 16 / sizeof(T);
  const int es = sizeof(T);
  const int vb = common_vec_bytes({reinterpret_cast<uintptr_t>(x), reinterpret_cast<uintptr_t>(y),
                                   ubytes(hw, es), ubytes(xsn, es),
                                   ubytes(xsb, es)});
  const int v = (vb >= 16) ? VMAX : 1;
  const uint64_t planes = static_cast<uint64_t>(mul_sat({n, b, c}));
  const uint64_t cpp = static_cast<uint64_t>(hw / v);
  const uint64_t total = static_cast<uint64_t>(mul_sat({static_cast<int64_t>(planes), static_cast<int64_t>(cpp)}));
  if (total >= 0x7fffffffull || cpp == 0) return set_error(WC_ERR_LIMIT, "wc_bn_eval: tensor too large");
  const dim3 grid(static_cast<uint32_t>(cdiv(total, kNormBlock)));
  const FastDiv fcpp = make_fastdiv(static_cast<uint32_t>(cpp));
  const FastDiv fc = make_fastdiv(static_cast<uint32_t>(c));
  const FastDiv fb = make_fastdiv(static_cast<uint32_t>(b));
  if (v == VMAX)
    bn_eval_kernel<T, P, VMAX><<<grid, kNormBlock, 0, st>>>(
        static_cast<const T*>(x), xsn, xsb, static_cast<const P*>(w), static_cast<const P*>(bias),
        static_cast<const P*>(rm), static_cast<const P*>(rv), eps, static_cast<T*>(y),
        static_cast<uint32_t>(total), fcpp, fc, fb, (int)hw, act == WC_ACT_RELU);
  else
    bn_eval_kernel<T, P, 1><<<grid, kNormBlock, 0, st>>>(
        static_cast<const T*>(x), xsn, xsb, static_cast<const P*>(w), static_cast<const P*>(bias),
        static_cast<const P*>(rm), static_cast<const P*>(rv), eps, static_cast<T*>(y),
        static_cast<uint32_t>(total), fcpp, fc, fb, (int)hw, act == WC_ACT_RELU);
  return check_launch("wc_bn_eval");
}

// ---------------------------------------------------------------------------
// GroupNorm / InstanceNorm.  A row is one (model, batch row, group): R = cpg * s
// contiguous elements of the N-first activation (cpg channels of s spatial
// elements).  WPR waves own a row; lane t of the row holds the V-element vectors
// (it * 64 WPR + t) for it < ITEMS in registers, so the row is read once and
// written once.  Statistics are two-pass fp32 (mean, then the mean squared
// deviation: the biased variance torch uses); one reciprocal square root per row.
// The affine weight of element e is that of channel g * cpg + e / s of its model
// (a vector never straddles two channels: s % V == 0).
// ---------------------------------------------------------------------------
struct GnParams {
  uint32_t rows;
  int r, s, cpg, c;
  FastDiv groups;       // row -> (model * batch + batch row, group)
  FastDiv per_model;    // row -> model (batch * groups rows per model)
  FastDiv sdiv;
  float eps;
  int relu;
};

template <int WPR>
__device__ __forceinline__ float gn_row_sum(float v, float* red) {
  v = group_reduce<64>(v);
  if constexpr (WPR == 1) {
    return v;
  } else {
    const int wave = threadIdx.x >> 6;
    __syncthreads();                      // red[] of the previous reduction has been read
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
  }
}

template <typename T, typename P, int V, int WPR, int ITEMS>
__global__ __launch_bounds__(kNormBlock) void groupnorm_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                              const P* __restrict__ w, const P* __restrict__ bias,
                                                              GnParams p) {
  constexpr int RPB = 4 / WPR;                           // rows per block
  constexpr int LT = 64 * WPR;                           // lanes per row
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const uint32_t row = blockIdx.x * RPB + (tid >> 6) / WPR;
  if (WPR == 1 && row >= p.rows) return;                 // whole waves leave together
  const bool live = row < p.rows;                        // (WPR == 4: one row per block)
  const int lt = tid & (LT - 1);
  const int64_t base = static_cast<int64_t>(live ? row : 0) * p.r;
  const T* xr = x + base;
  float v[ITEMS][V];
  float sum = 0.f;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int e = (it * LT + lt) * V;
    if (live && e < p.r) {
      LoadV<T, V>::ld(xr + e, v[it]);
#pragma unroll
      for (int k = 0; k < V; ++k) sum += v[it][k];
    } else {
#pragma unroll
      for (int k = 0; k < V; ++k) v[it][k] = 0.f;
    }
  }
  const float inv_r = 1.0f / static_cast<float>(p.r);
  const float mean = gn_row_sum<WPR>(sum, red) * inv_r;
  float sq = 0.f;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int e = (it * LT + lt) * V;
    if (e < p.r) {
#pragma unroll
      for (int k = 0; k < V; ++k) {
        const float d = v[it][k] - mean;
        sq += d * d;
      }
    }
  }
  const float rstd = 1.0f / sqrtf(gn_row_sum<WPR>(sq, red) * inv_r + p.eps);
  if (!live) return;
  const uint32_t mb = fdiv(row, p.groups);
  const int g = static_cast<int>(row - mb * p.groups.d);
  const uint32_t mdl = fdiv(row, p.per_model);
  const int64_t ch0 = static_cast<int64_t>(mdl) * p.c + g * p.cpg;
  T* yr = y + base;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int e = (it * LT + lt) * V;
    if (e < p.r) {
      const int64_t ch = ch0 + fdiv(static_cast<uint32_t>(e), p.sdiv);
      const float a = (w ? to_f32(w[ch]) : 1.f) * rstd;
      const float b = (bias ? to_f32(bias[ch]) : 0.f) - mean * a;
      float o[V];
#pragma unroll
      for (int k = 0; k < V; ++k) {
        o[k] = v[it][k] * a + b;
        if (p.relu) o[k] = fmaxf(o[k], 0.f);
      }
      LoadV<T, V>::st(yr + e, o);
    }
  }
}

// Rows longer than the register-resident configurations: one block per row,
// three passes over the row (sum, squared deviations, normalise).
template <typename T, typename P>
__global__ __launch_bounds__(kNormBlock) void groupnorm_long_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                                   const P* __restrict__ w,
                                                                   const P* __restrict__ bias, GnParams p) {
  __shared__ float red[4];
  const uint32_t row = blockIdx.x;
  const int64_t base = static_cast<int64_t>(row) * p.r;
  const T* xr = x + base;
  float sum = 0.f;
  for (int e = threadIdx.x; e < p.r; e += kNormBlock) sum += to_f32(xr[e]);
  const float inv_r = 1.0f / static_cast<float>(p.r);
  const float mean = gn_row_sum<4>(sum, red) * inv_r;
  float sq = 0.f;
  for (int e = threadIdx.x; e < p.r; e += kNormBlock) {
    const float d = to_f32(xr[e]) - mean;
    sq += d * d;
  }
  const float rstd = 1.0f / sqrtf(gn_row_sum<4>(sq, red) * inv_r + p.eps);
  const uint32_t mb = fdiv(row, p.groups);
  const int g = static_cast<int>(row - mb * p.groups.d);
  const uint32_t mdl = fdiv(row, p.per_model);
  const int64_t ch0 = static_cast<int64_t>(mdl) * p.c + g * p.cpg;
  T* yr = y + base;
  for (int e = threadIdx.x; e < p.r; e += kNormBlock) {
    const int64_t ch = ch0 + fdiv(static_cast<uint32_t>(e), p.sdiv);
    const float a = (w ? to_f32(w[ch]) : 1.f) * rstd;
    float o = (to_f32(xr[e]) - mean) * a + (bias ? to_f32(bias[ch]) : 0.f);
    if (p.relu) o = fmaxf(o, 0.f);
    yr[e] = from_f32<T>(o);
  }
}

template <typename T, typename P, int V>
int32_t launch_gn_v(const T* x, T* y, const P* w, const P* b, const GnParams& p, hipStream_t st) {
  const int r = p.r;
  auto go = [&](auto kern, int rows_per_block) {
    kern<<<dim3(static_cast<uint32_t>(cdiv(p.rows, rows_per_block))), kNormBlock, 0, st>>>(x, y, w, b, p);
    return check_launch("wc_group_norm");
  };
  if (r <= 64 * V * 1) return go(groupnorm_kernel<T, P, V, 1, 1>, 4);
  if (r <= 64 * V * 2) return go(groupnorm_kernel<T, P, V, 1, 2>, 4);
  if (r <= 64 * V * 4) return go(groupnorm_kernel<T, P, V, 1, 4>, 4);
  if (r <= 256 * V * 2) return go(groupnorm_kernel<T, P, V, 4, 2>, 1);
  if (r <= 256 * V * 4) return go(groupnorm_kernel<T, P, V, 4, 4>, 1);
  if (r <= 256 * V * 8) return go(groupnorm_kernel<T, P, V, 4, 8>, 1);
  if (V > 1 && r <= 256 * V * 16) return go(groupnorm_kernel<T, P, V, 4, 16>, 1);
  return go(groupnorm_long_kernel<T, P>, 1);
}

template <typename T, typename P>
int32_t launch_gn(const void* x, void* y, const void* w, const void* b, int64_t n, int64_t bt, int64_t c,
                  int64_t s, int64_t groups, float eps, int act, hipStream_t st) {
  constexpr int VMAX = 16 / sizeof(T);
  const int64_t cpg = c / groups;
  const int64_t r = mul_sat({cpg, s});
  const int64_t rows = mul_sat({n, bt, groups});
  if (r >= 0x7fffffffll || rows >= 0x7fffffffll || s >= 0x7fffffffll || mul_sat({n, c}) >= 0x7fffffffll)
    return set_error(WC_ERR_LIMIT, "wc_group_norm: tensor too large");
  GnParams p;
  p.rows = static_cast<uint32_t>(rows);
  p.r = static_cast<int>(r);
  p.s = static_cast<int>(s);
  p.cpg = static_cast<int>(cpg);
  p.c = static_cast<int>(c);
  p.groups = make_fastdiv(static_cast<uint32_t>(groups));
  p.per_model = make_fastdiv(static_cast<uint32_t>(bt * groups));
  p.sdiv = make_fastdiv(static_cast<uint32_t>(s));
  p.eps = eps;
  p.relu = act == WC_ACT_RELU;
  const T* xt = static_cast<const T*>(x);
  T* yt = static_cast<T*>(y);
  const P* wt = static_cast<const P*>(w);
  const P* bt_ = static_cast<const P*>(b);
  const bool vec = s % VMAX == 0 &&
                   common_vec_bytes({reinterpret_cast<uintptr_t>(x), reinterpret_cast<uintptr_t>(y)}) >= 16;
  return vec ? launch_gn_v<T, P, VMAX>(xt, yt, wt, bt_, p, st) : launch_gn_v<T, P, 1>(xt, yt, wt, bt_, p, st);
}

}  // namespace
}  // namespace wc

using namespace wc;

extern "C" int32_t wc_layernorm(const void* x, int64_t x_model_stride, int64_t x_row_stride,
                                const void* gamma, const void* beta, void* y,
                                int64_t y_model_stride, int64_t y_row_stride, int64_t n,
                                int64_t rows_per_model, int64_t dim, float eps, int32_t dtype,
                                int32_t param_dtype, void* stream) {
  clear_error();
  WC_REQUIRE(n >= 0 && rows_per_model >= 0 && dim >= 0, WC_ERR_SHAPE, "wc_layernorm: negative size");
  if (n == 0 || rows_per_model == 0 || dim == 0) return WC_OK;
  WC_REQUIRE(x && y && gamma, WC_ERR_NULL, "wc_layernorm: null pointer");
  WC_REQUIRE(mul_sat({n, rows_per_model}) < 0x7fffffffll, WC_ERR_LIMIT, "wc_layernorm: too many rows");
  WC_REQUIRE(dim < 0x7fffffffll, WC_ERR_LIMIT, "wc_layernorm: dim %lld too large", static_cast<long long>(dim));
  hipStream_t st = as_stream(stream);
  if (dtype == WC_F32 && param_dtype == WC_F32)
    return launch_layernorm<float, float>(x, x_model_stride, x_row_stride, gamma, beta, y,
                                          y_model_stride, y_row_stride, n, rows_per_model, dim, eps, st);
  if (dtype == WC_BF16 && param_dtype == WC_BF16)
    return launch_layernorm<bf16, bf16>(x, x_model_stride, x_row_stride, gamma, beta, y,
                                        y_model_stride, y_row_stride, n, rows_per_model, dim, eps, st);
  if (dtype == WC_BF16 && param_dtype == WC_F32)
    return launch_layernorm<bf16, float>(x, x_model_stride, x_row_stride, gamma, beta, y,
                                         y_model_stride, y_row_stride, n, rows_per_model, dim, eps, st);
  if (dtype == WC_F16 && param_dtype == WC_F16)
    return launch_layernorm<f16, f16>(x, x_model_stride, x_row_stride, gamma, beta, y,
                                      y_model_stride, y_row_stride, n, rows_per_model, dim, eps, st);
  return set_error(WC_ERR_DTYPE, "wc_layernorm: unsupported dtype pair (%s, %s)", dtype_name(dtype),
                   dtype_name(param_dtype));
}

extern "C" int32_t wc_embedding_layernorm(const void* weight, int64_t n, int64_t vocab, int64_t dim,
                                          const int64_t* ids, int64_t rows, int32_t ids_shared,
                                          const void* gamma, const void* beta, float eps, int32_t dtype,
                                          int32_t param_dtype, void* out, int32_t* err_flag, void* stream) {
  clear_error();
  WC_REQUIRE(n >= 0 && vocab >= 0 && dim >= 0 && rows >= 0, WC_ERR_SHAPE,
             "wc_embedding_layernorm: negative size");
  if (n == 0 || rows == 0 || dim == 0) return WC_OK;
  WC_REQUIRE(weight && ids && gamma && out, WC_ERR_NULL, "wc_embedding_layernorm: null pointer");
  WC_REQUIRE(rows < 0x7fffffffll && mul_sat({n, rows}) < 0x7fffffffll, WC_ERR_LIMIT,
             "wc_embedding_layernorm: too many rows");
  hipStream_t st = as_stream(stream);
  const int shared = ids_shared ? 1 : 0;
  if (dtype == WC_F32 && param_dtype == WC_F32)
    return launch_emb_layernorm<float, float>(weight, n, vocab, dim, ids, rows, shared, gamma, beta, eps, out,
                                              err_flag, st);
  if (dtype == WC_BF16 && param_dtype == WC_BF16)
    return launch_emb_layernorm<bf16, bf16>(weight, n, vocab, dim, ids, rows, shared, gamma, beta, eps, out,
                                            err_flag, st);
  if (dtype == WC_BF16 && param_dtype == WC_F32)
    return launch_emb_layernorm<bf16, float>(weight, n, vocab, dim, ids, rows, shared, gamma, beta, eps, out,
                                             err_flag, st);
  if (dtype == WC_F16 && param_dtype == WC_F16)
    return launch_emb_layernorm<f16, f16>(weight, n, vocab, dim, ids, rows, shared, gamma, beta, eps, out,
                                          err_flag, st);
  return set_error(WC_ERR_DTYPE, "wc_embedding_layernorm: unsupported dtype pair (%s, %s)", dtype_name(dtype),
                   dtype_name(param_dtype));
}

extern "C" int32_t wc_bn_eval(const void* x, int64_t x_stride_n, int64_t x_stride_b,
                              const void* weight, const void* bias, const void* running_mean,
                              const void* running_var, float eps, void* y, int64_t n, int64_t b,
                              int64_t c, int64_t hw, int32_t dtype, int32_t param_dtype,
                              int32_t act, void* stream) {
  clear_error();
  WC_REQUIRE(n >= 0 && b >= 0 && c >= 0 && hw >= 0, WC_ERR_SHAPE, "wc_bn_eval: negative size");
  if (n == 0 || b == 0 || c == 0 || hw == 0) return WC_OK;
  WC_REQUIRE(x && y && running_mean && running_var, WC_ERR_NULL, "wc_bn_eval: null pointer");
  WC_REQUIRE(act == WC_ACT_NONE || act == WC_ACT_RELU, WC_ERR_ARG, "wc_bn_eval: bad act %d", act);
  hipStream_t st = as_stream(stream);
  if (dtype == WC_F32 && param_dtype == WC_F32)
    return launch_bn<float, float>(x, x_stride_n, x_stride_b, weight, bias, running_mean,
                                   running_var, eps, y, n, b, c, hw, act, st);
  if (dtype == WC_BF16 && param_dtype == WC_BF16)
    return launch_bn<bf16, bf16>(x, x_stride_n, x_stride_b, weight, bias, running_mean,
                                 running_var, eps, y, n, b, c, hw, act, st);
  if (dtype == WC_BF16 && param_dtype == WC_F32)
    return launch_bn<bf16, float>(x, x_stride_n, x_stride_b, weight, bias, running_mean,
                                  running_var, eps, y, n, b, c, hw, act, st);
  if (dtype == WC_F16 && param_dtype == WC_F16)
    return launch_bn<f16, f16>(x, x_stride_n, x_stride_b, weight, bias, running_mean, running_var,
                               eps, y, n, b, c, hw, act, st);
  return set_error(WC_ERR_DTYPE, "wc_bn_eval: unsupported dtype pair (%s, %s)", dtype_name(dtype),
                   dtype_name(param_dtype));
}

extern "C" int32_t wc_group_norm(const void* x, void* y, int64_t n, int64_t b, int64_t c, int64_t s,
                                 int64_t groups, const void* weight, const void* bias, float eps,
                                 int32_t dtype, int32_t param_dtype, int32_t act, void* stream) {
  clear_error();
  WC_REQUIRE(n >= 0 && b >= 0 && c >= 0 && s >= 0, WC_ERR_SHAPE, "wc_group_norm: negative size");
  WC_REQUIRE(groups > 0 && c % groups == 0, WC_ERR_SHAPE, "wc_group_norm: %lld channels not divisible into %lld groups",
             (long long)c, (long long)groups);
  WC_REQUIRE(act == WC_ACT_NONE || act == WC_ACT_RELU, WC_ERR_ARG, "wc_group_norm: bad act %d", act);
  WC_REQUIRE((weight == nullptr) == (bias == nullptr), WC_ERR_ARG, "wc_group_norm: weight and bias go together");
  if (n == 0 || b == 0 || c == 0 || s == 0) return WC_OK;
  WC_REQUIRE(x && y, WC_ERR_NULL, "wc_group_norm: null pointer");
  hipStream_t st = as_stream(stream);
  if (dtype == WC_F32 && param_dtype == WC_F32)
    return launch_gn<float, float>(x, y, weight, bias, n, b, c, s, groups, eps, act, st);
  if (dtype == WC_BF16 && param_dtype == WC_BF16)
    return launch_gn<bf16, bf16>(x, y, weight, bias, n, b, c, s, groups, eps, act, st);
  if (dtype == WC_BF16 && param_dtype == WC_F32)
    return launch_gn<bf16, float>(x, y, weight, bias, n, b, c, s, groups, eps, act, st);
  if (dtype == WC_F16 && param_dtype == WC_F16)
    return launch_gn<f16, f16>(x, y, weight, bias, n, b, c, s, groups, eps, act, st);
  return set_error(WC_ERR_DTYPE, "wc_group_norm: unsupported dtype pair (%s, %s)", dtype_name(dtype),
                   dtype_name(param_dtype));
}
