// Two chained per-model Linear layers in one launch:
//   h[i][m] = act1( x[i][m] W1[i]^T + b1[i] )        (kept in LDS, never in HBM)
//   y[i][m] = act2( h[i][m] W2[i]^T + b2[i] )
// A workgroup (4 waves) owns 32 rows of one model, or 16 when 32-row workgroups would
// leave compute units idle (few models and rows): then all four waves share one 16-row
// block and split its column tiles four ways instead of two.  x rows, W1, W2 and h live in LDS
// as rows of 16-byte chunks, chunk q of row r stored at position q ^ (r & sw) (sw + 1
// a power of two dividing the row's chunk count), so the 16-byte fragment reads of
// consecutive rows hit distinct banks.  x, W1 and W2 are staged with LDS-DMA loads
// (global_load_lds_dwordx4: lane L of a wave writes 16 bytes at M0 + 16 L), so the
// whole ~70 KB of one workgroup is in flight at once with no register staging; the
// swizzle is applied on the global side (lane L fetches the chunk that belongs at its
// LDS position).  Both products are 16x16 MFMA tiles (bf16: v_mfma_f32_16x16x32_bf16,
// fp32: v_mfma_f32_16x16x4f32 with the 32-wide K block permuted so each lane reads 8
// consecutive values); each wave owns one 16-row block and computes its column tiles
// two at a time as independent accumulator chains with the next K block's fragments
// read ahead.  h is rounded to the element type before the second product, as a
// separate first layer would store it.
#include "wc_common.h"

namespace wc {
namespace {

constexpr int kMlpRows = 32;                     // rows per workgroup (at most)
constexpr int kMlpThreads = 256;
constexpr int kMlpMaxColBlocks = 16;             // hidden, out <= 256 (16-column blocks)

struct MlpParams {
  int n, m, in, hid, out;
  int act1, act2;
  int nin, nhid;                                 // 16-byte chunks per row of x / W1 and of h / W2
  int sw_in, sw_hid;                             // chunk swizzle masks
  FastDiv nin_d, nhid_d;
  const void* x;
  int64_t x_sn, x_so, x_si;
  FastDiv x_ri;
  const void* w1;
  const void* b1;
  const void* w2;
  const void* b2;
  void* y;
  int64_t y_sn, y_so, y_si;
  FastDiv y_ri;
  int row_blocks;
};

inline size_t mlp_lds_bytes(int es, int in, int hid, int out, int rows = kMlpRows) {
  return static_cast<size_t>(es) * (static_cast<size_t>(rows + hid) * in + static_cast<size_t>(rows + out) * hid);
}

// Largest power of two <= 16 dividing n, minus one (n a multiple of 8).
inline int mlp_swizzle_mask(int n) {
  int g = 16;
  while (n % g) g >>= 1;
  return g - 1;
}

__device__ __forceinline__ int mlp_pos(int r, int q, int n, int sw) { return r * n + (q ^ (r & sw)); }

// Stages a [rows][n] block of 16-byte chunks into LDS at `lds` (swizzled) with LDS-DMA
// loads.  row_src(r) is the global byte address of row r; the caller keeps every row
// it can name in bounds.  All loads are left in flight.
template <typename RowSrc>
__device__ __forceinline__ void mlp_dma(char* lds, int rows, int n, const FastDiv& nd, int sw, RowSrc row_src) {
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int lane = threadIdx.x & 63;
  const int total = rows * n;                    // a multiple of 64 (n % 8 == 0, rows % 16 == 0)
  for (int p0 = wave * 64; p0 < total; p0 += kMlpThreads) {
    const int pos = p0 + lane;
    const int r = static_cast<int>(fdiv(static_cast<uint32_t>(pos), nd));
    const int q = (pos - r * n) ^ (r & sw);      // the chunk that belongs at position pos
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(row_src(r) + q * 16), lds + p0 * 16, 16, 0, 0);
  }
}

// Fragments of one K block of 32 for a lane: bf16 one chunk, fp32 two (8 consecutive k).
template <typename T>
struct MlpFrag {
  using V = typename std::conditional<sizeof(T) == 2, bf16x8, f32x4>::type;
  V v[sizeof(T) == 2 ? 1 : 2];
};

template <typename T>
__device__ __forceinline__ MlpFrag<T> mlp_frag(const char* base, int n, int sw, int r, int k0) {
  MlpFrag<T> f;
  const int lane = threadIdx.x & 63;
  if constexpr (sizeof(T) == 2) {
    const int q = (k0 >> 3) + (lane >> 4);
    f.v[0] = *reinterpret_cast<const bf16x8*>(base + mlp_pos(r, q, n, sw) * 16);
  } else {
    const int q = (k0 >> 2) + (lane >> 4) * 2;
    f.v[0] = *reinterpret_cast<const f32x4*>(base + mlp_pos(r, q, n, sw) * 16);
    f.v[1] = *reinterpret_cast<const f32x4*>(base + mlp_pos(r, q + 1, n, sw) * 16);
  }
  return f;
}

template <typename T>
__device__ __forceinline__ f32x4 mlp_mma(const MlpFrag<T>& a, const MlpFrag<T>& b, f32x4 acc) {
  if constexpr (sizeof(T) == 2) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v[0], b.v[0], acc, 0, 0, 0);
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.v[h][s], b.v[h][s], acc, 0, 0, 0);
    return acc;
  }
}

// Two 16x16 tiles of A[ra.. ra+15] x B[rb0..]^T and A x B[rb1..]^T over K = k (a multiple
// of 32), as two interleaved accumulator chains; the next K block is read ahead (its
// index clamped, so the last read repeats a valid block).
template <typename T>
__device__ __forceinline__ void mlp_pair(const char* a, const char* b, int n, int sw, int k, int ra, int rb0, int rb1,
                                         f32x4& acc0, f32x4& acc1) {
  acc0 = f32x4{0.f, 0.f, 0.f, 0.f};
  acc1 = acc0;
  MlpFrag<T> fa = mlp_frag<T>(a, n, sw, ra, 0);
  MlpFrag<T> f0 = mlp_frag<T>(b, n, sw, rb0, 0);
  MlpFrag<T> f1 = mlp_frag<T>(b, n, sw, rb1, 0);
  for (int k0 = 0; k0 < k; k0 += 32) {
    const int kn = min(k0 + 32, k - 32);
    const MlpFrag<T> na = mlp_frag<T>(a, n, sw, ra, kn);
    const MlpFrag<T> n0 = mlp_frag<T>(b, n, sw, rb0, kn);
    const MlpFrag<T> n1 = mlp_frag<T>(b, n, sw, rb1, kn);
    if constexpr (sizeof(T) == 2) {
      acc0 = mlp_mma<T>(fa, f0, acc0);
      acc1 = mlp_mma<T>(fa, f1, acc1);
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(fa.v[h][s], f0.v[h][s], acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(fa.v[h][s], f1.v[h][s], acc1, 0, 0, 0);
        }
    }
    fa = na;
    f0 = n0;
    f1 = n1;
  }
}

// One 16x16 tile A[ra..ra+15] x B[rb..rb+15]^T over K = k: the column block left over
// when a wave's share of a layer's column blocks is odd.
template <typename T>
__device__ __forceinline__ void mlp_one(const char* a, const char* b, int n, int sw, int k, int ra, int rb,
                                        f32x4& acc) {
  acc = f32x4{0.f, 0.f, 0.f, 0.f};
  MlpFrag<T> fa = mlp_frag<T>(a, n, sw, ra, 0);
  MlpFrag<T> fb = mlp_frag<T>(b, n, sw, rb, 0);
  for (int k0 = 0; k0 < k; k0 += 32) {
    const int kn = min(k0 + 32, k - 32);
    const MlpFrag<T> na = mlp_frag<T>(a, n, sw, ra, kn);
    const MlpFrag<T> nb = mlp_frag<T>(b, n, sw, rb, kn);
    acc = mlp_mma<T>(fa, fb, acc);
    fa = na;
    fb = nb;
  }
}

// ROWS = 32: waves 0/1 and 2/3 take the two 16-row blocks, each pair splitting the column
// blocks two ways; ROWS = 16: the four waves split the one row block's column blocks.
template <typename T, int ROWS>
__global__ __launch_bounds__(kMlpThreads) void mlp2_kernel(MlpParams p) {
  static_assert(ROWS == 16 || ROWS == 32, "16 or 32 rows per workgroup");
  constexpr int RB = ROWS / 16;                  // row blocks per workgroup
  constexpr int CW = 4 / RB;                     // waves splitting a row block's column blocks
  constexpr int VE = 16 / sizeof(T);             // elements per 16-byte chunk
  extern __shared__ __attribute__((aligned(16))) char mlp_smem[];
  char* xs = mlp_smem;                                          // [ROWS][nin] chunks
  char* w1s = xs + ROWS * p.nin * 16;                           // [hid][nin]
  char* hs = w1s + p.hid * p.nin * 16;                          // [ROWS][nhid]
  char* w2s = hs + ROWS * p.nhid * 16;                          // [out][nhid]

  // Dispatch deals workgroups to the 8 XCDs in turn. With a grid of a multiple of 8, slot
  // b runs logical block (b % 8) * (grid / 8) + b / 8, so a model's consecutive row blocks
  // share one XCD's L2 and its weights are read from HBM once.
  int blk = static_cast<int>(blockIdx.x);
  if ((gridDim.x & 7) == 0) blk = (blk & 7) * static_cast<int>(gridDim.x >> 3) + (blk >> 3);
  const int mdl = blk / p.row_blocks;
  const int m0 = (blk - mdl * p.row_blocks) * ROWS;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int fr = lane & 15, rq = (lane >> 4) * 4;
  const int rbk = (wave % RB) * 16;              // the wave's 16-row block
  const int cg = wave / RB;                      // its column blocks: cg + CW i
  const int cb1 = p.hid / 16, cb2 = p.out / 16;  // column blocks per layer

  // biases of the lane's columns (block j = cg + CW i), read ahead of the staging
  float b1v[kMlpMaxColBlocks / 2], b2v[kMlpMaxColBlocks / 2];
  {
    const T* b1 = static_cast<const T*>(p.b1);
    const T* b2 = static_cast<const T*>(p.b2);
#pragma unroll
    for (int i = 0; i < kMlpMaxColBlocks / 2; ++i) {
      const int j = cg + CW * i;
      b1v[i] = b1 ? to_f32(b1[static_cast<int64_t>(mdl) * p.hid + min(j, cb1 - 1) * 16 + fr]) : 0.f;
      b2v[i] = b2 ? to_f32(b2[static_cast<int64_t>(mdl) * p.out + min(j, cb2 - 1) * 16 + fr]) : 0.f;
    }
  }

  // ---- stage x rows (rows past m repeat row m - 1; their outputs are not stored), W1, W2 ----
  {
    const char* xb = static_cast<const char*>(p.x) + static_cast<int64_t>(mdl) * p.x_sn * sizeof(T);
    const char* w1b = static_cast<const char*>(p.w1) + static_cast<int64_t>(mdl) * p.hid * p.in * sizeof(T);
    const char* w2b = static_cast<const char*>(p.w2) + static_cast<int64_t>(mdl) * p.out * p.hid * sizeof(T);
    const int last = p.m - 1;
    mlp_dma(xs, ROWS, p.nin, p.nin_d, p.sw_in, [&](int r) {
      const uint32_t gm = static_cast<uint32_t>(min(m0 + r, last));
      const uint32_t outer = fdiv(gm, p.x_ri);
      const uint32_t inner = gm - outer * p.x_ri.d;
      return xb + (static_cast<int64_t>(outer) * p.x_so + static_cast<int64_t>(inner) * p.x_si) * sizeof(T);
    });
    const int rb1 = p.nin * 16, rb2 = p.nhid * 16;
    mlp_dma(w1s, p.hid, p.nin, p.nin_d, p.sw_in, [&](int r) { return w1b + static_cast<int64_t>(r) * rb1; });
    mlp_dma(w2s, p.out, p.nhid, p.nhid_d, p.sw_hid, [&](int r) { return w2b + static_cast<int64_t>(r) * rb2; });
  }
  __builtin_amdgcn_s_waitcnt(0x70);              // vmcnt(0) lgkmcnt(0): this wave's chunks are in LDS
  __syncthreads();

  // ---- h = act1(x W1^T + b1) -> LDS (element type) ----
#pragma unroll
  for (int i = 0; i < kMlpMaxColBlocks / 2; i += 2) {
    const int j0 = cg + CW * i, j1 = j0 + CW;
    if (j0 >= cb1) break;
    const bool two = j1 < cb1;
    f32x4 acc[2];
    if (two)
      mlp_pair<T>(xs, w1s, p.nin, p.sw_in, p.in, rbk + fr, j0 * 16 + fr, j1 * 16 + fr, acc[0], acc[1]);
    else
      mlp_one<T>(xs, w1s, p.nin, p.sw_in, p.in, rbk + fr, j0 * 16 + fr, acc[0]);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      if (u == 1 && !two) break;
      const int col = (u ? j1 : j0) * 16 + fr;
      const float bv = b1v[i + u];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = rbk + rq + e;
        float v = acc[u][e] + bv;
        if (p.act1 == WC_ACT_RELU) v = fmaxf(v, 0.f);
        *reinterpret_cast<T*>(hs + mlp_pos(r, col / VE, p.nhid, p.sw_hid) * 16 + (col % VE) * sizeof(T)) =
            from_f32<T>(v);
      }
    }
  }
  __syncthreads();

  // ---- y = act2(h W2^T + b2) -> global ----
  T* yrow[4];
  bool live[4];
  {
    T* yb = static_cast<T*>(p.y) + static_cast<int64_t>(mdl) * p.y_sn;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int gm = m0 + rbk + rq + e;
      live[e] = gm < p.m;
      const uint32_t g = static_cast<uint32_t>(min(gm, p.m - 1));
      const uint32_t outer = fdiv(g, p.y_ri);
      const uint32_t inner = g - outer * p.y_ri.d;
      yrow[e] = yb + static_cast<int64_t>(outer) * p.y_so + static_cast<int64_t>(inner) * p.y_si;
    }
  }
#pragma unroll
  for (int i = 0; i < kMlpMaxColBlocks / 2; i += 2) {
    const int j0 = cg + CW * i, j1 = j0 + CW;
    if (j0 >= cb2) break;
    const bool two = j1 < cb2;
    f32x4 acc[2];
    if (two)
      mlp_pair<T>(hs, w2s, p.nhid, p.sw_hid, p.hid, rbk + fr, j0 * 16 + fr, j1 * 16 + fr, acc[0], acc[1]);
    else
      mlp_one<T>(hs, w2s, p.nhid, p.sw_hid, p.hid, rbk + fr, j0 * 16 + fr, acc[0]);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      if (u == 1 && !two) break;
      const int col = (u ? j1 : j0) * 16 + fr;
      const float bv = b2v[i + u];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = acc[u][e] + bv;
        if (p.act2 == WC_ACT_RELU) v = fmaxf(v, 0.f);
        if (live[e]) yrow[e][col] = from_f32<T>(v);
      }
    }
  }
}

}  // namespace
}  // namespace wc

using namespace wc;

extern "C" int32_t wc_mlp2_supported(int32_t dtype, int64_t in_features, int64_t hidden, int64_t out_features) {
  if (dtype != WC_F32 && dtype != WC_BF16) return 0;
  if (in_features <= 0 || hidden <= 0 || out_features <= 0) return 0;
  // rows of x / W1 and of h / W2 are whole groups of 8 16-byte chunks (fp32: 32 elements,
  // bf16: 64); out is whole 16-column tiles; at most kMlpMaxColBlocks column blocks per layer
  const int64_t grain = dtype == WC_F32 ? 32 : 64;
  if (in_features % grain || hidden % grain || out_features % 16) return 0;
  if (hidden > 16 * kMlpMaxColBlocks || out_features > 16 * kMlpMaxColBlocks || in_features > 4096) return 0;
  const size_t lds = mlp_lds_bytes(dtype_size(dtype), (int)in_features, (int)hidden, (int)out_features);
  return lds <= 160 * 1024 ? 1 : 0;
}

extern "C" int32_t wc_mlp2(const wc_mlp2_args* a, void* stream) {
  clear_error();
  WC_REQUIRE(a != nullptr, WC_ERR_NULL, "wc_mlp2: null args");
  WC_REQUIRE(a->n >= 0 && a->m >= 0, WC_ERR_SHAPE, "wc_mlp2: negative size");
  WC_REQUIRE(wc_mlp2_supported(a->dtype, a->in_features, a->hidden, a->out_features), WC_ERR_LIMIT,
             "wc_mlp2: sizes %lld -> %lld -> %lld (%s) not supported by the fused kernel",
             (long long)a->in_features, (long long)a->hidden, (long long)a->out_features, dtype_name(a->dtype));
  WC_REQUIRE(a->act1 == WC_ACT_NONE || a->act1 == WC_ACT_RELU, WC_ERR_ARG, "wc_mlp2: bad act1");
  WC_REQUIRE(a->act2 == WC_ACT_NONE || a->act2 == WC_ACT_RELU, WC_ERR_ARG, "wc_mlp2: bad act2");
  if (a->n == 0 || a->m == 0) return WC_OK;
  WC_REQUIRE(a->x && a->w1 && a->w2 && a->y, WC_ERR_NULL, "wc_mlp2: null pointer");
  WC_REQUIRE(a->x_rows_inner > 0 && a->y_rows_inner > 0, WC_ERR_ARG, "wc_mlp2: rows_inner must be positive");
  WC_REQUIRE(a->x_rows_inner < 0x7fffffffll && a->y_rows_inner < 0x7fffffffll, WC_ERR_LIMIT,
             "wc_mlp2: rows_inner too large");
  WC_REQUIRE(a->m < 0x7fffffffll && a->n < 0x7fffffffll, WC_ERR_LIMIT, "wc_mlp2: sizes too large");
  const int es = dtype_size(a->dtype);
  WC_REQUIRE(common_vec_bytes({reinterpret_cast<uintptr_t>(a->x), reinterpret_cast<uintptr_t>(a->w1),
                               reinterpret_cast<uintptr_t>(a->w2), ubytes(a->x_stride_n, es),
                               ubytes(a->x_stride_outer, es),
                               ubytes(a->x_stride_inner, es)}) >= 16,
             WC_ERR_ALIGN, "wc_mlp2: x / weight rows must be 16-byte aligned");
  MlpParams p;
  p.n = (int)a->n;
  p.m = (int)a->m;
  p.in = (int)a->in_features;
  p.hid = (int)a->hidden;
  p.out = (int)a->out_features;
  p.act1 = a->act1;
  p.act2 = a->act2;
  p.x = a->x;
  p.x_sn = a->x_stride_n;
  p.x_so = a->x_stride_outer;
  p.x_si = a->x_stride_inner;
  p.x_ri = make_fastdiv(static_cast<uint32_t>(a->x_rows_inner));
  p.nin = p.in * es / 16;
  p.nhid = p.hid * es / 16;
  p.nin_d = make_fastdiv(static_cast<uint32_t>(p.nin));
  p.nhid_d = make_fastdiv(static_cast<uint32_t>(p.nhid));
  p.sw_in = mlp_swizzle_mask(p.nin);
  p.sw_hid = mlp_swizzle_mask(p.nhid);
  p.w1 = a->w1;
  p.b1 = a->b1;
  p.w2 = a->w2;
  p.b2 = a->b2;
  p.y = a->y;
  p.y_sn = a->y_stride_n;
  p.y_so = a->y_stride_outer;
  p.y_si = a->y_stride_inner;
  p.y_ri = make_fastdiv(static_cast<uint32_t>(a->y_rows_inner));
  // 16-row workgroups when 32-row ones would not cover the compute units
  const int cus = device_cu_count();
  const int rows = static_cast<int64_t>(p.n) * cdiv(p.m, kMlpRows) < cus ? 16 : kMlpRows;
  p.row_blocks = static_cast<int>(cdiv(p.m, rows));
  const int64_t blocks = static_cast<int64_t>(p.n) * p.row_blocks;
  WC_REQUIRE(blocks < 0x7fffffffll, WC_ERR_LIMIT, "wc_mlp2: too many blocks");
  hipStream_t st = as_stream(stream);
  const bool f32 = a->dtype == WC_F32;
  const size_t lds = mlp_lds_bytes(es, p.in, p.hid, p.out, rows);
  const void* kern = rows == 16 ? (f32 ? reinterpret_cast<const void*>(mlp2_kernel<float, 16>)
                                       : reinterpret_cast<const void*>(mlp2_kernel<bf16, 16>))
                                : (f32 ? reinterpret_cast<const void*>(mlp2_kernel<float, kMlpRows>)
                                       : reinterpret_cast<const void*>(mlp2_kernel<bf16, kMlpRows>));
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess)
      return set_error(static_cast<int32_t>(e), "wc_mlp2: LDS of %zu bytes refused: %s", lds, hipGetErrorString(e));
  }
  const dim3 grid(static_cast<uint32_t>(blocks));
  if (rows == 16) {
    if (f32)
      mlp2_kernel<float, 16><<<grid, kMlpThreads, lds, st>>>(p);
    else
      mlp2_kernel<bf16, 16><<<grid, kMlpThreads, lds, st>>>(p);
  } else {
    if (f32)
      mlp2_kernel<float, kMlpRows><<<grid, kMlpThreads, lds, st>>>(p);
    else
      mlp2_kernel<bf16, kMlpRows><<<grid, kMlpThreads, lds, st>>>(p);
  }
  return check_launch("wc_mlp2");
}
