// Implicit-GEMM grouped convolution (N independent Conv1d / Conv2d layers) on
// MFMA with a fused epilogue:
//   y[i,b,co,p] = act( BN_i,co( sum_{ci,r,s} x[i,b,ci,p@(r,s)] W[i,co,ci,r,s] + bias )
//                      + R[i,b,co,p] )
// Per model the GEMM is  M = output pixels, N = C_out, K = C_in * kh * kw.
//
// Workgroup = (model, image, pixel tile, 64-channel output tile), 4 waves.
//  * The input tile (output tile + halo) is staged once in LDS as
//    channels-last [row][col][ci] with a padded channel pitch, so an MFMA A
//    fragment (8 consecutive input channels of one pixel) is one 16-byte LDS
//    read, and the tile is reused by all kh*kw taps.
//  * Weights are pre-packed (wc_conv_pack_weights) to [N, C_out, kh, kw, Ci32]
//    so a B fragment (8 consecutive input channels of one tap and one output
//    channel) is one 16-byte load that stays resident in L2/L1; B fragments of
//    the next K-step are fetched while the current one runs.
//  * Each wave computes FM x 4 MFMA tiles (FM*16 pixels x 64 channels): every
//    A fragment feeds four MFMAs.
//  * Epilogue: bias, eval-BatchNorm folded as (v * alpha + beta), written to
//    LDS as [co][pixel] in the output type, then residual add + ReLU during
//    coalesced NCHW stores.
#include "wc_common.h"

namespace wc {
namespace {

struct ConvParams {
  int n, batch, ci, co, h, w, kh, kw, sh, sw, ph, pw, dh, dw, ho, wo;
  // depth of a 3-D convolution (2-D: kd = d = dout = 1, sd = dd = 1, pd = 0); only the
  // general kernel reads them.  x_cs / y_cs: channel-plane strides (d*h*w, dout*ho*wo).
  int kd, sd, pd, dd, d, dout;
  int64_t x_cs, y_cs;
  int ci32;                 // input channels padded to a multiple of 32
  int cc;                   // input channels staged per LDS chunk (multiple of 32)
  int tr, tc;               // output tile rows / cols
  int ir, ic;               // input tile rows / cols
  int tiles_r, tiles_c, tiles_co;
  int remap, act, vec_out;
  FastDiv fd_plane, fd_ic;  // ir*ic and ic
  const void* x;
  int64_t x_sn, x_sb;
  const void* wp;           // packed weights [n][co][kh][kw][ci32]
  const void* wn;           // or (resident-weight kernel only) the filter bank [n*co][ci][kh][kw]
  const void* bias;         // [n*co] or null
  const void* bn_w;         // eval BN params [n*co] (bn_mean null: no BN)
  const void* bn_b;
  const void* bn_mean;
  const void* bn_var;
  float bn_eps;
  int pdt;                  // element type of bias / BN params
  const void* res;
  int64_t r_sn, r_sb;
  void* y;
  int64_t y_sn, y_sb;
};

constexpr int kConvThreads = 256;
constexpr int kFN = 4;            // 16-wide MFMA tiles along output channels (64)

__device__ __forceinline__ float ldp(const void* p, int dt, int64_t i) {
  if (dt == WC_F32) return static_cast<const float*>(p)[i];
  if (dt == WC_F16) return static_cast<float>(static_cast<const f16*>(p)[i]);
  return static_cast<float>(static_cast<const bf16*>(p)[i]);
}

template <typename T> struct ConvTraits;
// Tile sizes keep one workgroup's LDS near 50 KB so three workgroups share a CU
// and hide each other's global-memory latency.
template <> struct ConvTraits<bf16> {
  static constexpr int kFM = 4;    // 64 pixels per wave, 256 per tile
  static constexpr int kPad = 8;   // channel pitch padding (elements)
};
template <> struct ConvTraits<f16> {
  static constexpr int kFM = 4;
  static constexpr int kPad = 8;
};
template <> struct ConvTraits<float> {
  static constexpr int kFM = 2;    // 32 pixels per wave, 128 per tile
  static constexpr int kPad = 4;
};

// Epilogue shared by the conv kernels (LDS free on entry): bias + folded eval
// BatchNorm into LDS as [co][pixel] in the output type, then residual add +
// ReLU during coalesced NCHW stores.
// Per-lane folded bias / eval-BatchNorm affine of the 4 output channels
// j * 16 + (lane & 15) the lane writes: y = acc * alpha + beta.
__device__ __forceinline__ void conv_affine(const ConvParams& p, int mdl, int co0, float (&alpha)[kFN],
                                            float (&beta)[kFN]) {
  const int fr = threadIdx.x & 15;
#pragma unroll
  for (int j = 0; j < kFN; ++j) {
    const int co = co0 + j * 16 + fr;
    alpha[j] = 1.f;
    beta[j] = 0.f;
    if (co < p.co) {
      const int64_t pi = static_cast<int64_t>(mdl) * p.co + co;
      const float bv = p.bias ? ldp(p.bias, p.pdt, pi) : 0.f;
      if (p.bn_mean) {
        const float inv = 1.0f / sqrtf(ldp(p.bn_var, p.pdt, pi) + p.bn_eps);
        alpha[j] = p.bn_w ? inv * ldp(p.bn_w, p.pdt, pi) : inv;
        beta[j] = (p.bn_b ? ldp(p.bn_b, p.pdt, pi) : 0.f) - ldp(p.bn_mean, p.pdt, pi) * alpha[j];
        beta[j] += bv * alpha[j];   // (acc + bias) * alpha + beta
      } else {
        beta[j] = bv;
      }
    }
  }
}

template <typename T, int FM>
__device__ __forceinline__ void conv_epilogue(const ConvParams& p, const f32x4 (&acc)[FM][kFN], T* xs, int mdl,
                                              int bb, int ho0, int wo0, int co0, const float (&alpha)[kFN],
                                              const float (&beta)[kFN], int od = 0) {
  constexpr int TPIX = 4 * FM * 16;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int fr = lane & 15;
  // ---- epilogue 1: bias + folded BN, into LDS as [co][pixel] (type T) ----
  constexpr int CPITCH = TPIX + 8;
  T* cs = xs;  // reuse the input tile buffer
#pragma unroll
  for (int j = 0; j < kFN; ++j) {
    const int col = j * 16 + fr;          // output channel within the tile
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int px = wave * FM * 16 + i * 16 + (lane >> 4) * 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) cs[col * CPITCH + px + e] = from_f32<T>(acc[i][j][e] * alpha[j] + beta[j]);
    }
  }
  __syncthreads();

  // ---- epilogue 2: residual + activation, coalesced NCHW stores ----
  const int64_t dpl = static_cast<int64_t>(od) * p.ho * p.wo;   // output depth slice
  T* yb = static_cast<T*>(p.y) + mdl * p.y_sn + bb * p.y_sb + dpl;
  const T* rb = p.res ? static_cast<const T*>(p.res) + mdl * p.r_sn + bb * p.r_sb + dpl : nullptr;
  const int64_t how = p.y_cs;                                    // channel-plane stride
  constexpr int VE = 16 / sizeof(T);
  if (p.vec_out) {
    // tc % VE == 0, wo0 % VE == 0, rows of y / res 16-byte aligned; EB chunks per
    // thread are handled together so their residual loads are in flight at once
    constexpr int EB = 4;
    const int chunks = 64 * (TPIX / VE);
    for (int e0 = tid; e0 < chunks; e0 += EB * kConvThreads) {
      int64_t off[EB];
      int lds_at[EB];
      uint4 rv[EB];
#pragma unroll
      for (int u = 0; u < EB; ++u) {
        const int e = e0 + u * kConvThreads;
        off[u] = -1;
        if (e >= chunks) continue;
        const int col = e / (TPIX / VE);
        const int px = (e - col * (TPIX / VE)) * VE;
        const int pr = px / p.tc, pc = px - (px / p.tc) * p.tc;
        const int co = co0 + col, oh = ho0 + pr, ow = wo0 + pc;
        if (co >= p.co || pr >= p.tr || oh >= p.ho || ow >= p.wo) continue;
        off[u] = static_cast<int64_t>(co) * how + oh * p.wo + ow;
        lds_at[u] = col * CPITCH + px;
        if (rb) rv[u] = *reinterpret_cast<const uint4*>(rb + off[u]);
      }
#pragma unroll
      for (int u = 0; u < EB; ++u) {
        if (off[u] < 0) continue;
        float v[VE];
        const T* src = &cs[lds_at[u]];
#pragma unroll
        for (int q = 0; q < VE; ++q) v[q] = to_f32(src[q]);
        if (rb) {
          const T* rr = reinterpret_cast<const T*>(&rv[u]);
#pragma unroll
          for (int q = 0; q < VE; ++q) v[q] = to_f32(from_f32<T>(v[q] + to_f32(rr[q])));
        }
        uint4 ov;
        T* oo = reinterpret_cast<T*>(&ov);
#pragma unroll
        for (int q = 0; q < VE; ++q) oo[q] = from_f32<T>(p.act == WC_ACT_RELU ? fmaxf(v[q], 0.f) : v[q]);
        *reinterpret_cast<uint4*>(yb + off[u]) = ov;
      }
    }
  } else {
    for (int e = tid; e < 64 * TPIX; e += kConvThreads) {
      const int col = e / TPIX;
      const int px = e - col * TPIX;
      const int pr = px / p.tc, pc = px - (px / p.tc) * p.tc;
      const int co = co0 + col, oh = ho0 + pr, ow = wo0 + pc;
      if (co >= p.co || pr >= p.tr || oh >= p.ho || ow >= p.wo) continue;
      const int64_t off = static_cast<int64_t>(co) * how + oh * p.wo + ow;
      float v = to_f32(cs[col * CPITCH + px]);
      if (rb) v = to_f32(from_f32<T>(v + to_f32(rb[off])));
      if (p.act == WC_ACT_RELU) v = fmaxf(v, 0.f);
      yb[off] = from_f32<T>(v);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kConvThreads) void conv_kernel(ConvParams p) {
  constexpr int FM = ConvTraits<T>::kFM;
  constexpr int PAD = ConvTraits<T>::kPad;
  extern __shared__ float4 smem4[];
  T* xs = reinterpret_cast<T*>(smem4);
  const int cip = p.cc + PAD;                         // LDS channel pitch

  // ---- tile coordinates ----
  const int per_img = p.tiles_r * p.tiles_c * p.tiles_co;
  const int nblk = p.n * p.batch * p.dout * per_img;
  int bid = blockIdx.x;
  if (p.remap) bid = (blockIdx.x & 7) * (nblk >> 3) + (blockIdx.x >> 3);
  const int img = bid / per_img;                      // (model, image, output depth)
  int rem = bid - img * per_img;
  const int tco = rem / (p.tiles_r * p.tiles_c);
  rem -= tco * (p.tiles_r * p.tiles_c);
  const int trr = rem / p.tiles_c;
  const int tcc = rem - trr * p.tiles_c;
  const int mdl = img / (p.batch * p.dout);
  const int bd = img - mdl * (p.batch * p.dout);
  const int bb = bd / p.dout;
  const int od = bd - bb * p.dout;
  const int ho0 = trr * p.tr, wo0 = tcc * p.tc, co0 = tco * 64;
  const int hi0 = ho0 * p.sh - p.ph, wi0 = wo0 * p.sw - p.pw;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int fr = lane & 15, fk = (lane >> 4) * 8;

  const T* xb = static_cast<const T*>(p.x) + mdl * p.x_sn + bb * p.x_sb;
  const int taps_all = p.kd * p.kh * p.kw;
  const T* wb = static_cast<const T*>(p.wp) + static_cast<int64_t>(mdl) * p.co * taps_all * p.ci32;

  // LDS offset (elements, tap (0,0), channel fk) of each A-fragment pixel
  int aoff[FM];
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int px = wave * FM * 16 + i * 16 + fr;
    const int pr = px / p.tc, pc = px - (px / p.tc) * p.tc;
    const bool ok = pr < p.tr;
    aoff[i] = ok ? ((pr * p.sh) * p.ic + pc * p.sw) * cip + fk : fk;
  }
  // B-fragment weight rows (output channel per j) and their validity
  const T* wrow[kFN];
#pragma unroll
  for (int j = 0; j < kFN; ++j) {
    const int co = co0 + j * 16 + fr;
    wrow[j] = (co < p.co) ? wb + static_cast<int64_t>(co) * taps_all * p.ci32 + fk : nullptr;
  }

  f32x4 acc[FM][kFN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < kFN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int taps = p.kh * p.kw;
  bool staged = false;
  // depth taps (one for 2-D): input depth slice di; slices outside the input add zero
  for (int t = 0; t < p.kd; ++t) {
  const int di = od * p.sd - p.pd + t * p.dd;
  if (di < 0 || di >= p.d) continue;                  // uniform over the workgroup
  for (int c0 = 0; c0 < p.ci32; c0 += p.cc) {
    // ---- stage input channels [c0, c0+cc) of the tile as [row][col][ci] ----
    // unit = (group of 8 channels, tile pixel): 8 loads (consecutive lanes read
    // consecutive pixels of one channel plane -> coalesced), one 16-byte LDS store.
    if (staged) __syncthreads();
    staged = true;
    {
      const int plane = p.ir * p.ic;
      const int units = (p.cc >> 3) * plane;
      constexpr int U = 8;   // units per thread in flight: all loads issued before the stores
      for (int e0 = tid; e0 < units; e0 += U * kConvThreads) {
        T v[U][8];
        int dst[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int e = e0 + u * kConvThreads;
          dst[u] = -1;
          if (e < units) {
            const int cg = static_cast<int>(fdiv(static_cast<uint32_t>(e), p.fd_plane));
            const int rc = e - cg * plane;
            const int r = static_cast<int>(fdiv(static_cast<uint32_t>(rc), p.fd_ic));
            const int col = rc - r * p.ic;
            const int hi = hi0 + r, wi = wi0 + col, ch0 = c0 + cg * 8;
            const bool in = hi >= 0 && hi < p.h && wi >= 0 && wi < p.w;
            const T* src = xb + static_cast<int64_t>(ch0) * p.x_cs + (static_cast<int64_t>(di) * p.h + hi) * p.w + wi;
            const int64_t cstride = p.x_cs;
#pragma unroll
            for (int q = 0; q < 8; ++q)
              v[u][q] = (in && ch0 + q < p.ci) ? src[q * cstride] : from_f32<T>(0.f);
            dst[u] = rc * cip + cg * 8;
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (dst[u] < 0) continue;
          if constexpr (sizeof(T) == 2) {
            *reinterpret_cast<uint4*>(&xs[dst[u]]) = *reinterpret_cast<const uint4*>(v[u]);
          } else {
            *reinterpret_cast<uint4*>(&xs[dst[u]]) = *reinterpret_cast<const uint4*>(v[u]);
            *reinterpret_cast<uint4*>(&xs[dst[u] + 4]) = *reinterpret_cast<const uint4*>(v[u] + 4);
          }
        }
      }
    }
    __syncthreads();

    const int ksteps = taps * (p.cc / 32);
    // B fragments for K-step 0 of this chunk
    auto bload = [&](int ks, uint4* dst) {
      const int tap = ks / (p.cc / 32);
      const int cs = ks - tap * (p.cc / 32);
      const int64_t koff = static_cast<int64_t>(t * taps + tap) * p.ci32 + c0 + cs * 32;
#pragma unroll
      for (int j = 0; j < kFN; ++j) {
        if (sizeof(T) == 2) {
          dst[2 * j] = wrow[j] ? *reinterpret_cast<const uint4*>(wrow[j] + koff) : make_uint4(0, 0, 0, 0);
        } else {
          dst[2 * j] = wrow[j] ? *reinterpret_cast<const uint4*>(wrow[j] + koff) : make_uint4(0, 0, 0, 0);
          dst[2 * j + 1] = wrow[j] ? *reinterpret_cast<const uint4*>(wrow[j] + koff + 4) : make_uint4(0, 0, 0, 0);
        }
      }
    };
    uint4 bcur[2 * kFN], bnxt[2 * kFN];
    bload(0, bcur);
    for (int ks = 0; ks < ksteps; ++ks) {
      if (ks + 1 < ksteps) bload(ks + 1, bnxt);
      const int tap = ks / (p.cc / 32);
      const int cs = ks - tap * (p.cc / 32);
      const int r = tap / p.kw, s = tap - (tap / p.kw) * p.kw;
      const int toff = ((r * p.dh) * p.ic + s * p.dw) * cip + cs * 32;
      if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const bf16x8 a = *reinterpret_cast<const bf16x8*>(&xs[aoff[i] + toff]);
#pragma unroll
          for (int j = 0; j < kFN; ++j)
            acc[i][j] = mma16<T>(a, *reinterpret_cast<const bf16x8*>(&bcur[2 * j]), acc[i][j]);
        }
      } else {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const float* ap = reinterpret_cast<const float*>(&xs[aoff[i] + toff]);
          const f32x4 a0 = *reinterpret_cast<const f32x4*>(ap);
          const f32x4 a1 = *reinterpret_cast<const f32x4*>(ap + 4);
#pragma unroll
          for (int j = 0; j < kFN; ++j) {
            const f32x4 b0 = *reinterpret_cast<const f32x4*>(&bcur[2 * j]);
            const f32x4 b1 = *reinterpret_cast<const f32x4*>(&bcur[2 * j + 1]);
#pragma unroll
            for (int q = 0; q < 4; ++q)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[q], b0[q], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int q = 0; q < 4; ++q)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1[q], b1[q], acc[i][j], 0, 0, 0);
          }
        }
      }
      if (ks + 1 < ksteps) {
#pragma unroll
        for (int q = 0; q < 2 * kFN; ++q) bcur[q] = bnxt[q];
      }
    }
  }
  }

  float alpha[kFN], beta[kFN];
  conv_affine(p, mdl, co0, alpha, beta);
  __syncthreads();
  conv_epilogue<T, FM>(p, acc, xs, mdl, bb, ho0, wo0, co0, alpha, beta, od);
}

// ---------------------------------------------------------------------------
// Fast path (bf16, stride 1, W % 8 == 0, at most kFastTaps taps): per
// 32-channel chunk, BOTH operands are staged in LDS -- the input tile
// [row][col][ci] and the packed weights [tap][co][ci] -- so the K loop is LDS
// reads + MFMAs only.  The NCHW input is read as 16-byte vectors of 8 pixels
// of one channel; a thread loads 8 channels x 8 pixels and transposes them in
// registers into 8 pixel vectors of 8 channels (one 16-byte LDS store each).
// Halo cells outside the image are zero-filled.  Two workgroups share a CU.
// ---------------------------------------------------------------------------
constexpr int kFastTaps = 9;
constexpr int kFCC = 32;                // channels per chunk
constexpr int kFPitch = kFCC + 8;       // LDS channel pitch (elements): 80 bytes

// 8x8 transpose of bf16: in[q] = 8 pixels of channel q -> out[p] = 8 channels of pixel p
// (component access only, so the arrays stay in registers)
__device__ __forceinline__ uint32_t dword_of(const u32x4& v, int i) { return v[i]; }

__device__ __forceinline__ void transpose8x8_bf16(const u32x4 (&in)[8], u32x4 (&out)[8]) {
#pragma unroll
  for (int px = 0; px < 8; ++px) {
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t a = dword_of(in[2 * j], px >> 1), b = dword_of(in[2 * j + 1], px >> 1);
      o[j] = (px & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
    }
    out[px] = u32x4{o[0], o[1], o[2], o[3]};
  }
}

template <typename PT>
__device__ __forceinline__ float ldpt(const void* p, int64_t i) {
  return to_f32(static_cast<const PT*>(p)[i]);
}

// Persistent form of the fast path.  One workgroup per CU walks a contiguous
// range of work items (model, 64-channel output tile, image, pixel tile),
// ordered so that neighbouring items share the model's weights.  Each item is
// processed in stages of 32 input channels; a stage's operands (input tile
// chunk [row][col][ci] and weight chunk [tap][co][ci]) live in one of two LDS
// buffers, and the next stage's global loads are in flight during the current
// stage's MFMAs.  The item's epilogue reuses the LDS buffer it just finished.
struct Stage {
  int mdl, bb, tco, ho0, wo0, c0;
};

// KT: compile-time tap count (0: runtime), so 3x3 convolutions get a fully
// unrolled tap loop whose LDS reads are scheduled ahead of the MFMAs.
template <typename PT, bool PERSIST, int KT>
__global__ __launch_bounds__(kConvThreads, PERSIST ? 1 : 2) void conv_persist_kernel(ConvParams p, int per_wg,
                                                                                   int extra) {
  using T = bf16;
  constexpr int FM = 4;                               // 64 pixels per wave
  extern __shared__ float4 smem4[];
  const int taps = KT ? KT : p.kh * p.kw;
  const int in_elems = p.ir * p.ic * kFPitch;
  const int stage_elems = in_elems + taps * 64 * kFPitch;
  T* lds0 = reinterpret_cast<T*>(smem4);
  T* trash = lds0 + (PERSIST ? 2 : 1) * stage_elems; // 16-byte sink for masked-off stores

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int fr = lane & 15, fk = (lane >> 4) * 8;
  const int nch = p.ci32 / kFCC;
  const int tiles_img = p.tiles_r * p.tiles_c;
  const int64_t plane = static_cast<int64_t>(p.h) * p.w;
  int w = blockIdx.x;
  if (!PERSIST && p.remap) w = (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
  const int i_begin = PERSIST ? w * per_wg + (w < extra ? w : extra) : w;
  const int n_items = PERSIST ? per_wg + (w < extra ? 1 : 0) : 1;
  const int S = n_items * nch;
  const u32x4 z4 = u32x4{0u, 0u, 0u, 0u};

  auto stage_of = [&](int s) {
    Stage st;
    const int item = i_begin + s / nch;
    st.c0 = (s - (s / nch) * nch) * kFCC;
    const int t = item % tiles_img;
    int rest = item / tiles_img;
    st.bb = rest % p.batch;
    rest /= p.batch;
    st.tco = rest % p.tiles_co;
    st.mdl = rest / p.tiles_co;
    const int trr = t / p.tiles_c;
    st.ho0 = trr * p.tr;
    st.wo0 = (t - trr * p.tiles_c) * p.tc;
    return st;
  };

  // pixel offsets of this lane's A fragments within an input tile
  int aoff[FM];
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int px = wave * FM * 16 + i * 16 + fr;
    const int pr = px / p.tc, pc = px - (px / p.tc) * p.tc;
    aoff[i] = (pr < p.tr ? (pr * p.ic + pc) * kFPitch : 0) + fk;
  }
  // weight pieces of this thread: (co, tap, 8-channel group), fixed over stages
  constexpr int kWPT = kFastTaps * 64 * (kFCC / 8) / kConvThreads;
  const int wpieces = 64 * taps * (kFCC / 8);
  int wco[kWPT], wtq[kWPT], wdst[kWPT];
#pragma unroll
  for (int q = 0; q < kWPT; ++q) {
    const int e0 = tid + q * kConvThreads;
    const int e = e0 < wpieces ? e0 : wpieces - 1;
    wco[q] = e / (taps * 4);
    wtq[q] = e - wco[q] * (taps * 4);                   // tap * 4 + channel group
    wdst[q] = e0 < wpieces ? in_elems + ((wtq[q] >> 2) * 64 + wco[q]) * kFPitch + (wtq[q] & 3) * 8 : -1;
  }

  // ---- stage registers and their issue / commit ----
  u32x4 wreg[kWPT], xreg[8];
  struct XBlk { int cg, r, v; bool row_ok; } xb_cur;
  auto xblock = [&](const Stage& st, int e, XBlk& blk, int& hic, int& vclamp, int& v0, int& nv) {
    const int hi0 = st.ho0 - p.ph, wi0 = st.wo0 - p.pw;
    const int c_lo = wi0 > 0 ? wi0 : 0;
    const int c_hi = (wi0 + p.ic < p.w) ? wi0 + p.ic : p.w;
    v0 = c_lo >> 3;
    nv = c_hi > c_lo ? ((c_hi + 7) >> 3) - v0 : 0;
    const int blocks = (kFCC / 8) * p.ir * nv;
    const int ee = (e < blocks) ? e : 0;
    blk.cg = nv ? ee / (p.ir * nv) : 0;
    const int r2 = nv ? ee - blk.cg * (p.ir * nv) : 0;
    blk.r = nv ? r2 / nv : 0;
    blk.v = v0 + (nv ? r2 - blk.r * nv : 0);
    const int hi = hi0 + blk.r;
    blk.row_ok = e < blocks && hi >= 0 && hi < p.h;
    hic = hi < 0 ? 0 : (hi >= p.h ? p.h - 1 : hi);
    vclamp = blk.v * 8 + 8 <= p.w ? blk.v : (p.w >> 3) - 1;
    return blocks;
  };
  auto issue = [&](const Stage& st) {
    const T* wb = static_cast<const T*>(p.wp) + static_cast<int64_t>(st.mdl) * p.co * taps * p.ci32;
    const int co0 = st.tco * 64;
#pragma unroll
    for (int q = 0; q < kWPT; ++q) {
      const int co = co0 + wco[q] < p.co ? co0 + wco[q] : p.co - 1;
      wreg[q] = *reinterpret_cast<const u32x4*>(wb + (static_cast<int64_t>(co) * taps + (wtq[q] >> 2)) * p.ci32 +
                                                 st.c0 + (wtq[q] & 3) * 8);
    }
    int hic, vcl, v0, nv;
    xblock(st, tid, xb_cur, hic, vcl, v0, nv);
    const T* xbase = static_cast<const T*>(p.x) + st.mdl * p.x_sn + st.bb * p.x_sb;
    const int ch0 = st.c0 + xb_cur.cg * 8;
    const T* src = xbase + static_cast<int64_t>(hic) * p.w + vcl * 8;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int ch = ch0 + q < p.ci ? ch0 + q : p.ci - 1;
      xreg[q] = *reinterpret_cast<const u32x4*>(src + ch * plane);
    }
  };
  auto store_block = [&](T* buf, const Stage& st, int cg, int r, int v, bool row_ok, const u32x4 (&in)[8]) {
    const int wi0 = st.wo0 - p.pw;
    u32x4 out[8];
    transpose8x8_bf16(in, out);
#pragma unroll
    for (int px = 0; px < 8; ++px) {
      const int col = v * 8 + px - wi0;
      const bool ok = row_ok && col >= 0 && col < p.ic;
      T* dst = ok ? buf + (r * p.ic + col) * kFPitch + cg * 8 : trash;
      *reinterpret_cast<u32x4*>(dst) = out[px];
    }
  };
  auto commit = [&](T* buf, const Stage& st) {
    const int co0 = st.tco * 64;
#pragma unroll
    for (int q = 0; q < kWPT; ++q) {
      T* dst = wdst[q] >= 0 ? buf + wdst[q] : trash;
      *reinterpret_cast<u32x4*>(dst) = (wdst[q] >= 0 && co0 + wco[q] < p.co) ? wreg[q] : z4;
    }
    int hic, vcl, v0, nv;
    const int blocks = xblock(st, tid, xb_cur, hic, vcl, v0, nv);
    {
      const int ch0 = st.c0 + xb_cur.cg * 8;
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (!(xb_cur.row_ok && ch0 + q < p.ci)) xreg[q] = z4;
      store_block(buf, st, xb_cur.cg, xb_cur.r, xb_cur.v, xb_cur.row_ok, xreg);
    }
    // further rounds of input blocks (wide tiles only): load and store directly
    const T* xbase = static_cast<const T*>(p.x) + st.mdl * p.x_sn + st.bb * p.x_sb;
    for (int e = tid + kConvThreads; e < blocks; e += kConvThreads) {
      XBlk blk;
      int hic2, vcl2, v02, nv2;
      xblock(st, e, blk, hic2, vcl2, v02, nv2);
      const int ch0 = st.c0 + blk.cg * 8;
      u32x4 in[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int ch = ch0 + q < p.ci ? ch0 + q : p.ci - 1;
        const u32x4 t = *reinterpret_cast<const u32x4*>(xbase + ch * plane + static_cast<int64_t>(hic2) * p.w +
                                                        vcl2 * 8);
        in[q] = (blk.row_ok && ch0 + q < p.ci) ? t : z4;
      }
      store_block(buf, st, blk.cg, blk.r, blk.v, blk.row_ok, in);
    }
    // zero halo cells outside the image
    const int hi0 = st.ho0 - p.ph, wi0 = st.wo0 - p.pw;
    const int cells = p.ir * p.ic;
    for (int e = tid; e < cells * (kFCC / 8); e += kConvThreads) {
      const int cg = e / cells;
      const int cell = e - cg * cells;
      const int r = cell / p.ic, col = cell - (cell / p.ic) * p.ic;
      const int hi = hi0 + r, wi = wi0 + col;
      if (hi < 0 || hi >= p.h || wi < 0 || wi >= p.w)
        *reinterpret_cast<u32x4*>(buf + cell * kFPitch + cg * 8) = z4;
    }
  };

  // bias / BN parameters of an item, loaded with straight-line code
  float pv[5][kFN];
  auto load_params = [&](const Stage& st) {
    const void* dummy = p.wp;
    const void* ptrs[5] = {p.bias ? p.bias : dummy, p.bn_w ? p.bn_w : dummy, p.bn_b ? p.bn_b : dummy,
                           p.bn_mean ? p.bn_mean : dummy, p.bn_var ? p.bn_var : dummy};
#pragma unroll
    for (int j = 0; j < kFN; ++j) {
      const int co = st.tco * 64 + j * 16 + fr;
      const int64_t pi = static_cast<int64_t>(st.mdl) * p.co + (co < p.co ? co : p.co - 1);
#pragma unroll
      for (int k = 0; k < 5; ++k) pv[k][j] = ldpt<PT>(ptrs[k], pi);
    }
  };
  auto fold_params = [&](float (&alpha)[kFN], float (&beta)[kFN]) {
#pragma unroll
    for (int j = 0; j < kFN; ++j) {
      const float bv = p.bias ? pv[0][j] : 0.f;
      if (p.bn_mean) {
        const float inv = 1.0f / sqrtf(pv[4][j] + p.bn_eps);
        alpha[j] = p.bn_w ? inv * pv[1][j] : inv;
        beta[j] = (p.bn_b ? pv[2][j] : 0.f) - pv[3][j] * alpha[j] + bv * alpha[j];
      } else {
        alpha[j] = 1.f;
        beta[j] = bv;
      }
    }
  };

  f32x4 acc[FM][kFN];
  if (S > 0) {
    Stage cur = stage_of(0);
    if (!PERSIST) load_params(cur);                   // one item: its parameters arrive with the first stage
    issue(cur);
    commit(lds0, cur);
  }
  __syncthreads();
  for (int s = 0; s < S; ++s) {
    const Stage cur = stage_of(s);
    T* buf = lds0 + (PERSIST ? (s & 1) * stage_elems : 0);
    const bool more = s + 1 < S;
    const Stage nxt = stage_of(more ? s + 1 : s);
    // (persistent) this item's bias / BN parameters: loaded every stage before
    // the prefetch, so waiting for them never waits for the prefetch
    if (PERSIST) load_params(cur);
    issue(nxt);                                       // unconditional: see the fast kernel
    if (cur.c0 == 0) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < kFN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // ---- K loop: taps x 32 channels, both operands from LDS ----
    const T* wsm = buf + in_elems;
#pragma unroll
    for (int tap = 0; tap < (KT ? KT : taps); ++tap) {
      const int r = tap / p.kw, sc = tap - (tap / p.kw) * p.kw;
      const int toff = (r * p.dh * p.ic + sc * p.dw) * kFPitch;
      const T* wt = wsm + tap * 64 * kFPitch + fr * kFPitch + fk;
      bf16x8 bfr[kFN];
#pragma unroll
      for (int j = 0; j < kFN; ++j) bfr[j] = *reinterpret_cast<const bf16x8*>(wt + j * 16 * kFPitch);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(buf + aoff[i] + toff);
#pragma unroll
        for (int j = 0; j < kFN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bfr[j], acc[i][j], 0, 0, 0);
      }
    }
    __syncthreads();                                  // everyone is done reading buf
    if (PERSIST && cur.c0 + kFCC >= p.ci32) {
      // last chunk of the item: epilogue through buf (it has an internal barrier)
      float alpha[kFN], beta[kFN];
      fold_params(alpha, beta);
      conv_epilogue<T, FM>(p, acc, buf, cur.mdl, cur.bb, cur.ho0, cur.wo0, cur.tco * 64, alpha, beta);
    }
    if (more) commit(lds0 + (PERSIST ? ((s + 1) & 1) * stage_elems : 0), nxt);
    __syncthreads();
  }
  if (!PERSIST && S > 0) {
    // single item: its epilogue runs after the last stage, through the stage buffer
    const Stage cur = stage_of(S - 1);
    float alpha[kFN], beta[kFN];
    fold_params(alpha, beta);
    conv_epilogue<T, FM>(p, acc, lds0, cur.mdl, cur.bb, cur.ho0, cur.wo0, cur.tco * 64, alpha, beta);
  }
}

// ---------------------------------------------------------------------------
// Resident-weight "same" convolution (bf16, stride 1, dilation 1, pad k/2,
// C_in in {32, 64}, C_out % 64 == 0, width W with 256 / W output rows per
// item).  A persistent workgroup walks a contiguous range of items (model,
// 64-channel output tile, image, row block):
//  * the weights of the current (model, channel tile) stay in LDS as
//    [tap][co][ci] and are reloaded only when the range crosses into the next
//    model or channel tile;
//  * LDS rows are 16-byte chunks of 8 channels whose chunk index is XOR-
//    swizzled by the pixel (or output channel) index, so the 16 lanes that
//    read one MFMA fragment row hit 16 distinct bank groups without padding;
//  * every LDS address of the K loop is a per-lane base plus a compile-time
//    offset, and the fragments of K-step s + 1 are read during step s.
// Two groups of 4 waves (one wave of each group per SIMD) take alternate
// items and alternate roles every phase: while one group runs the MFMA loop of
// its item out of its own input buffer, the other finishes its previous item
// (bias, folded eval BatchNorm, residual, ReLU; 8-byte stores of 4 pixels)
// and stages its next item: NCHW 16-byte vectors loaded one phase earlier are
// transposed 8x8 in registers into the channels-last swizzled layout.  So on
// every SIMD one wave issues MFMAs while the other's VALU work and memory
// waits overlap them.  Global accesses are buffer operations whose
// out-of-range lanes the hardware drops (stores) or reads as zero (loads:
// rows outside the image, items past the range).
// ---------------------------------------------------------------------------
template <int KH, int KW, int CI, int W>
struct ResConv {
  static constexpr int TR = 256 / W;                 // output rows per item
  static constexpr int IR = TR + KH - 1;             // staged input rows
  static constexpr int IC = W + KW - 1;              // staged input cols (halo cols are zero)
  static constexpr int PH = KH / 2, PW = KW / 2;
  static constexpr int PXB = CI * 2;                 // bytes per staged pixel
  static constexpr int NCH = CI / 8;                 // 16-byte chunks per pixel
  static constexpr int PPB = 256 / PXB;              // pixels per 256-byte bank row
  static constexpr int TAPS = KH * KW;
  static constexpr int KS = CI / 32;                 // MFMA k-steps per tap
  static constexpr int STEPS = TAPS * KS;
  static constexpr int W_BYTES = TAPS * 64 * PXB;    // resident weights
  static constexpr int IN_BYTES = IR * IC * PXB;     // one input buffer (one per group)
  static constexpr int PAR_BYTES = 64 * 2 * 4;       // folded (alpha, beta) of the 64 output channels
  static constexpr int LDS = W_BYTES + 2 * IN_BYTES + PAR_BYTES;
  static constexpr int VPR = W / 8;                  // 16-byte vectors per input row and channel
  static constexpr int UNITS = NCH * IR * VPR;       // staging units (8 channels x 8 pixels)
  static constexpr int UPT = (UNITS + 255) / 256;    // staging units per thread of a group
  static_assert(256 % W == 0 && W >= 16, "width");
  static_assert(CI == 32 || CI == 64, "channels");
  static_assert(LDS <= 160 * 1024, "LDS");
  __device__ static constexpr int swz(int chunk, int idx) { return chunk ^ ((idx / PPB) & (NCH - 1)); }
};

struct ResItem {
  int mdl, tco, b, th;
};

constexpr uint32_t kResOob = 0x80000000u;            // buffer offset of a dropped / zero lane

// A buffer descriptor over one (model, batch row) block of `bytes` bytes: offsets past it
// (kResOob included) read zero / store nothing.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t res_rsrc(const void* base, int32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// 8x8 bf16 transpose with v_perm_b32: in[q] = 8 pixels of channel q -> out[x] =
// 8 channels of pixel x
__device__ __forceinline__ void transpose8x8_perm(const u32x4 (&in)[8], u32x4 (&out)[8]) {
#pragma unroll
  for (int x = 0; x < 8; ++x) {
    const uint32_t sel = (x & 1) ? 0x07060302u : 0x05040100u;
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = __builtin_amdgcn_perm(in[2 * j + 1][x >> 1], in[2 * j][x >> 1], sel);
    out[x] = u32x4{o[0], o[1], o[2], o[3]};
  }
}

template <int KH, int KW, int CI, int W, typename PT>
__global__ __launch_bounds__(512, 1) void conv_res_kernel(ConvParams p, int per_wg, int extra) {
  using C = ResConv<KH, KW, CI, W>;
  constexpr int TR = C::TR, IR = C::IR, IC = C::IC, PXB = C::PXB, NCH = C::NCH, TAPS = C::TAPS, KS = C::KS;
  constexpr int STEPS = C::STEPS;
  extern __shared__ __attribute__((aligned(16))) char lds[];
  char* const wlds = lds;                              // [tap][64 co][CI] swizzled
  char* const ilds = lds + C::W_BYTES;                 // 2 x [IR][IC][CI] swizzled, buffer g for group g
  float* const plds = reinterpret_cast<float*>(lds + C::W_BYTES + 2 * C::IN_BYTES);   // [64][alpha, beta]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2, wl = wave & 3;            // group, wave within the group
  const int gtid = tid & 255;
  const int fr = lane & 15, kq = lane >> 4;
  const int th_n = (p.ho + TR - 1) / TR;
  const int wg = blockIdx.x;
  const int i_begin = wg * per_wg + (wg < extra ? wg : extra);
  const int count = per_wg + (wg < extra ? 1 : 0);
  if (count <= 0) return;
  const u32x4 z4 = u32x4{0u, 0u, 0u, 0u};

  auto decode = [&](int t) {                           // local item t of this workgroup
    ResItem it;
    const int item = i_begin + t;
    it.th = item % th_n;
    int r = item / th_n;
    it.b = r % p.batch;
    r /= p.batch;
    it.tco = r % p.tiles_co;
    it.mdl = r / p.tiles_co;
    return it;
  };

  // ---- zero the halo columns of input buffers b0..b1-1 (staging never writes them) ----
  auto zero_halo = [&](int b0, int b1) {
    for (int e = tid; e < (b1 - b0) * IR * (KW - 1) * NCH; e += 512) {
      const int chunk = e % NCH;
      int r = e / NCH;
      const int hc = r % (KW - 1);
      r /= (KW - 1);
      const int row = r % IR, buf = b0 + r / IR;
      const int col = hc < C::PW ? hc : W + hc;
      *reinterpret_cast<u32x4*>(ilds + buf * C::IN_BYTES + (row * IC + col) * PXB + chunk * 16) = z4;
    }
  };
  zero_halo(0, 2);

  // ---- staging: NCHW 16-byte vectors -> registers -> channels-last LDS ----
  // unit u = (channel group cg fastest, 16-byte column vector v, staged row ir)
  uint32_t xoff[C::UPT];                               // byte offset of (channel cg*8, row 0, vector v)
  int xrow[C::UPT];
#pragma unroll
  for (int k = 0; k < C::UPT; ++k) {
    const int u = gtid + k * 256;
    const int cg = u % NCH, rest = u / NCH;
    const int v = rest % C::VPR, ir = rest / C::VPR;
    xrow[k] = u < C::UNITS ? ir : -0x40000000;         // never inside the image
    xoff[k] = static_cast<uint32_t>((cg * 8 * p.h) * W + v * 8) * 2u;
  }
  const uint32_t cstride = static_cast<uint32_t>(p.h * W) * 2u;   // channel plane bytes
  u32x4 xr[C::UPT][8];
  auto load_input = [&](int t) {
    const bool valid = t < count;
    const ResItem it = decode(valid ? t : 0);
    const __amdgpu_buffer_rsrc_t rs =
        res_rsrc(static_cast<const bf16*>(p.x) + it.mdl * p.x_sn + it.b * p.x_sb, CI * p.h * W * 2);
    const int r0 = it.th * TR - C::PH;
#pragma unroll
    for (int k = 0; k < C::UPT; ++k) {
      const int row = r0 + xrow[k];
      const bool ok = valid && row >= 0 && row < p.h;
      const uint32_t base = xoff[k] + static_cast<uint32_t>(row * W) * 2u;
#pragma unroll
      for (int q = 0; q < 8; ++q)
        xr[k][q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, ok ? base + q * cstride : kResOob,
                                                                                   0, 0));
    }
  };
  auto store_input = [&]() {
    char* base = ilds + grp * C::IN_BYTES;
    // the LDS addresses are recomputed per call (an opaque copy of the thread index
    // keeps the compiler from holding 8 of them per unit live across phases)
    int g_op = gtid;
    asm volatile("" : "+v"(g_op));
#pragma unroll
    for (int k = 0; k < C::UPT; ++k) {
      const int u = g_op + k * 256;
      if (k + 1 < C::UPT || C::UNITS % 256 == 0 || u < C::UNITS) {   // (only a partial last round branches)
        const int cg = u % NCH, rest = u / NCH;
        const int v = rest % C::VPR, ir = rest / C::VPR;
        u32x4 t[8];
        transpose8x8_perm(xr[k], t);
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          const int col = C::PW + v * 8 + x;
          *reinterpret_cast<u32x4*>(base + (ir * IC + col) * PXB + C::swz(cg, col) * 16) = t[x];
        }
      }
    }
  };

  // ---- resident weights (all 512 threads) ----
  auto load_weights = [&](const ResItem& it) {
    // 16-byte pieces in global order; all loads are issued before the LDS stores so
    // their latencies overlap
    constexpr int PIECES = TAPS * 64 * NCH;
    constexpr int PPT = (PIECES + 511) / 512;
    u32x4 v[PPT];
    // addresses are recomputed from an opaque copy of the thread index at every call, so
    // the compiler does not keep them live (in registers the K loop needs) between calls
    int t_op = tid;
    asm volatile("" : "+v"(t_op));
    if (p.wn) {
      // the filter bank as the module holds it, [n*co][ci][kh][kw]: input channels
      // chunk*8 .. chunk*8+7 of output channel co are 8 * TAPS contiguous elements
      // ([ci][tap]), which thread (co, chunk) loads as TAPS 16-byte vectors and transposes in
      // registers into one 16-byte piece per tap (channel k of tap t is element k*TAPS + t)
      constexpr int PAIRS = 64 * NCH;
      static_assert(PAIRS <= 512, "one (co, chunk) pair per thread");
      if (t_op < PAIRS) {
        const int chunk = t_op % NCH, co = t_op / NCH;
        const u32x4* src = reinterpret_cast<const u32x4*>(
            static_cast<const bf16*>(p.wn) +
            ((static_cast<int64_t>(it.mdl) * p.co + it.tco * 64 + co) * CI + chunk * 8) * TAPS);
        uint32_t in[TAPS * 4];
#pragma unroll
        for (int t = 0; t < TAPS; ++t) {
          const u32x4 a = src[t];
#pragma unroll
          for (int w = 0; w < 4; ++w) in[t * 4 + w] = a[w];
        }
        char* const dst = wlds + co * PXB + C::swz(chunk, co) * 16;
#pragma unroll
        for (int t = 0; t < TAPS; ++t) {
          uint32_t o[4];
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const int m0 = 2 * w * TAPS + t, m1 = m0 + TAPS;   // low and high halves of word w
            const uint32_t sel = ((m0 & 1) ? 0x0302u : 0x0100u) | ((m1 & 1) ? 0x07060000u : 0x05040000u);
            o[w] = __builtin_amdgcn_perm(in[m1 >> 1], in[m0 >> 1], sel);
          }
          *reinterpret_cast<u32x4*>(dst + t * 64 * PXB) = u32x4{o[0], o[1], o[2], o[3]};
        }
      }
    } else {
      // packed [n][co][tap][ci]: pieces ordered (co, tap, chunk)
      const bf16* wb = static_cast<const bf16*>(p.wp) +
                       (static_cast<int64_t>(it.mdl) * p.co + it.tco * 64) * TAPS * CI;
#pragma unroll
      for (int q = 0; q < PPT; ++q) {
        const int e = t_op + q * 512;
        v[q] = e < PIECES ? *reinterpret_cast<const u32x4*>(wb + static_cast<int64_t>(e) * 8) : z4;
      }
#pragma unroll
      for (int q = 0; q < PPT; ++q) {
        const int e = t_op + q * 512;
        if (e < PIECES) {
          const int chunk = e % NCH;
          const int rest = e / NCH;
          const int tap = rest % TAPS, co = rest / TAPS;
          *reinterpret_cast<u32x4*>(wlds + (tap * 64 + co) * PXB + C::swz(chunk, co) * 16) = v[q];
        }
      }
    }
    // folded per-channel affine of the epilogue: y = acc * alpha + beta
    if (tid < 64) {
      const int64_t pi = static_cast<int64_t>(it.mdl) * p.co + it.tco * 64 + tid;
      const float bv = p.bias ? ldpt<PT>(p.bias, pi) : 0.f;
      float a = 1.f, b = bv;
      if (p.bn_mean) {
        const float inv = 1.0f / sqrtf(ldpt<PT>(p.bn_var, pi) + p.bn_eps);
        a = p.bn_w ? inv * ldpt<PT>(p.bn_w, pi) : inv;
        b = (p.bn_b ? ldpt<PT>(p.bn_b, pi) : 0.f) - ldpt<PT>(p.bn_mean, pi) * a + bv * a;
      }
      plds[2 * tid] = a;
      plds[2 * tid + 1] = b;
    }
  };

  // ---- per-lane LDS bases of the K loop ----
  // A (input pixels): lane row fr of MFMA tile i is output pixel wl*64 + i*16 + fr
  // of the item; tap (r, s) reads staged pixel (pr + r, pc + s).
  const int px0 = wl * 64 + fr;
  const int pr0 = px0 / W, pc0 = px0 % W;
  int abase[KW][KS];
#pragma unroll
  for (int s = 0; s < KW; ++s)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      abase[s][ks] = C::W_BYTES + grp * C::IN_BYTES + (pr0 * IC + pc0 + s) * PXB + C::swz(ks * 4 + kq, pc0 + s) * 16;
  auto aoff_i = [](int i) { return ((i * 16) / W * IC + (i * 16) % W) * PXB; };
  int bbase[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) bbase[ks] = fr * PXB + C::swz(ks * 4 + kq, fr) * 16;

  // ---- output / residual byte offsets.  The epilogue regroups each 16-channel tile
  // j so that one 16-byte store per lane covers whole 128-byte runs (the wave's 64
  // pixels) of 8 channels: the lane stores 8 pixels starting at pixel wl*64 + 8 g
  // of the item, of channel j*16 + (fr & ~1) (store A) and the next channel
  // (store B, one channel plane further) ----
  const int how = p.ho * W;
  const int g_st = 4 * (fr & 1) + 2 * (kq & 1) + (kq >> 1);
  const uint32_t lane_off = static_cast<uint32_t>((fr & ~1) * how + wl * 64 + 8 * g_st) * 2u;
  const int lane_orow = (wl * 64 + 8 * g_st) / W;
  const uint32_t plane = static_cast<uint32_t>(how) * 2u;
  const float relu_floor = p.act == WC_ACT_RELU ? 0.f : -__builtin_huge_valf();
  const bool has_res = p.res != nullptr;

  // ---- state of this group's item between its compute and finish phases ----
  f32x4 acc[4][kFN];
  float alpha[kFN], beta[kFN];
  ResItem fin_it = {0, 0, 0, 0};

  auto compute = [&](int t) {
    const ResItem it = decode(t);
#pragma unroll
    for (int j = 0; j < kFN; ++j) {                     // this item's folded affine (LDS, loaded with the weights)
      alpha[j] = plds[2 * (j * 16 + fr)];
      beta[j] = plds[2 * (j * 16 + fr) + 1];
    }
    fin_it = it;
    // K loop: taps x k-steps, both operands from LDS.  B fragments are double-
    // buffered (step s + 1's are read at the start of step s); the A fragment of
    // row tile i is re-read for step s + 1 right after its last MFMA of step s,
    // 16 MFMAs ahead of its next use.
    bf16x8 fa[4], fb[2][kFN];
    auto b_load = [&](int step, bf16x8 (&b)[kFN]) {
      const int tap = step / KS, ks = step % KS;
#pragma unroll
      for (int j = 0; j < kFN; ++j)
        b[j] = *reinterpret_cast<const bf16x8*>(wlds + bbase[ks] + (tap * 64 + j * 16) * PXB);
    };
    auto a_load = [&](int step, int i) {
      const int tap = step / KS, ks = step % KS;
      const int r = tap / KW, s = tap % KW;
      fa[i] = *reinterpret_cast<const bf16x8*>(lds + abase[s][ks] + r * IC * PXB + aoff_i(i));
    };
    b_load(0, fb[0]);
#pragma unroll
    for (int i = 0; i < 4; ++i) a_load(0, i);
#pragma unroll
    for (int step = 0; step < STEPS; ++step) {
      const int c = step & 1;
      if (step + 1 < STEPS) b_load(step + 1, fb[c ^ 1]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < kFN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fb[c][j],
                                                               step == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[i][j],
                                                               0, 0, 0);
        if (step + 1 < STEPS) a_load(step + 1, i);
      }
      if (step + 1 < STEPS) {
        __builtin_amdgcn_sched_group_barrier(0x100, kFN, 0);   // next step's B fragments
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, kFN, 0); // row tile i's MFMAs
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // then its next A fragment
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Finish the group's last computed item, two channel tiles at a time: residual loads
  // first (their latency overlaps the staging work in between), then affine (+ ReLU),
  // the regrouping, residual + ReLU and the stores.
  //
  // Regrouping of tile j.  After the MFMAs lane (fr, kq) holds channel j*16 + fr at
  // pixels i*16 + kq*4 + [0, 4) of the wave's 64 (row tiles i = 0..3), packed to bf16
  // pairs: X = tiles 0, 2 and Y = tiles 1, 3.  (1) a 16-lane-row swap exchanges X of
  // the odd 16-lane rows (kq = 1, 3) with Y of the even rows, so every lane holds two
  // 8-pixel chunks of its channel, chunk s = {X[2s], X[2s+1], Y[2s], Y[2s+1]} at
  // pixels 8 (4 s + 2 (kq & 1) + (kq >> 1)).  (2) Lanes fr and fr ^ 1 (a DPP quad
  // permutation) trade chunks, so the even lane holds chunk 0 of both channels and
  // the odd lane chunk 1 of both: store A writes channel fr & ~1, store B channel
  // fr | 1, each as 8 lanes x 16 contiguous bytes.
  uint4 rv[2][2];                                       // residual chunks (A, B) of two tiles
  auto res_issue = [&](int j0) {
    const ResItem& it = fin_it;
    const __amdgpu_buffer_rsrc_t rrs =
        res_rsrc(static_cast<const bf16*>(p.res) + it.mdl * p.r_sn + it.b * p.r_sb, p.co * how * 2);
    const uint32_t obase = static_cast<uint32_t>(it.tco * 64 * how + it.th * TR * W) * 2u;
    const int left = p.ho - it.th * TR;
    const uint32_t off = lane_orow < (left < TR ? left : TR) ? lane_off : kResOob;
#pragma unroll
    for (int j = j0; j < j0 + 2; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        rv[j - j0][h] = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(rrs, off, obase + static_cast<uint32_t>(j * 32 * how) + h * plane, 0));
  };
  auto finish = [&](auto res, int j0) {
    constexpr bool kRes = decltype(res)::value;
    const ResItem& it = fin_it;
    const __amdgpu_buffer_rsrc_t yrs =
        res_rsrc(static_cast<bf16*>(p.y) + it.mdl * p.y_sn + it.b * p.y_sb, p.co * how * 2);
    const uint32_t obase = static_cast<uint32_t>(it.tco * 64 * how + it.th * TR * W) * 2u;
    const int left = p.ho - it.th * TR;
    const uint32_t off = lane_orow < (left < TR ? left : TR) ? lane_off : kResOob;
    const bool odd = fr & 1;
#pragma unroll
    for (int j = j0; j < j0 + 2; ++j) {
      uint32_t xy[2][4];                                // [X, Y][tile pair, bf16 pair]
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float v0 = acc[i][j][2 * h] * alpha[j] + beta[j];
          float v1 = acc[i][j][2 * h + 1] * alpha[j] + beta[j];
          if constexpr (!kRes) {
            v0 = fmaxf(v0, relu_floor);
            v1 = fmaxf(v1, relu_floor);
          }
          xy[i & 1][(i >> 1) * 2 + h] = pack_bf16x2(v0, v1);
        }
      // (1) as a lane-crossbar shuffle: v_permlane16_swap here gave wrong words now and then
      // (timing-dependent; the compiler's wait states around it did not cover it)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const bool odd_row = (kq & 1) != 0;
        const uint32_t recv = static_cast<uint32_t>(__shfl_xor(static_cast<int>(odd_row ? xy[0][k] : xy[1][k]), 16, 64));
        if (odd_row)
          xy[0][k] = recv;
        else
          xy[1][k] = recv;
      }
      uint32_t va[4], vb[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t c0 = xy[k >> 1][k & 1], c1 = xy[k >> 1][2 + (k & 1)];
        const uint32_t recv = static_cast<uint32_t>(
            __builtin_amdgcn_update_dpp(0, static_cast<int>(odd ? c0 : c1), 0xB1, 0xF, 0xF, true));
        va[k] = odd ? recv : c0;
        vb[k] = odd ? c1 : recv;
      }
      if constexpr (kRes) {
        const uint32_t* ra = reinterpret_cast<const uint32_t*>(&rv[j - j0][0]);
        const uint32_t* rb = reinterpret_cast<const uint32_t*>(&rv[j - j0][1]);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          va[k] = pack_bf16x2(fmaxf(bf16_lo(va[k]) + bf16_lo(ra[k]), relu_floor),
                              fmaxf(bf16_hi(va[k]) + bf16_hi(ra[k]), relu_floor));
          vb[k] = pack_bf16x2(fmaxf(bf16_lo(vb[k]) + bf16_lo(rb[k]), relu_floor),
                              fmaxf(bf16_hi(vb[k]) + bf16_hi(rb[k]), relu_floor));
        }
      }
      const uint32_t sb = obase + static_cast<uint32_t>(j * 32 * how);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, make_uint4(va[0], va[1], va[2], va[3])), yrs, off,
                                             sb, 0);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, make_uint4(vb[0], vb[1], vb[2], vb[3])), yrs, off,
                                             sb + plane, 0);
    }
  };

  auto lds_barrier = [&]() {
    __builtin_amdgcn_s_waitcnt(0xc07f);                 // lgkmcnt(0): this wave's LDS writes landed
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  // Phases 0..count: in phase t group t & 1 computes item t while the other group
  // finishes item t - 1 and stages item t + 1.  Each group runs its own straight
  // sequence (compute, barrier, finish + stage, barrier, ...), group 1 one phase
  // behind; both pass count + 1 barriers, and after each the weights of the
  // next phase's item are loaded if they change.
  int ph = 0;
  auto phase_end = [&]() {
    lds_barrier();
    if (ph + 1 < count) {
      const ResItem a = decode(ph), b = decode(ph + 1);
      if (a.mdl != b.mdl || a.tco != b.tco) {
        load_weights(b);
        __syncthreads();
      }
    }
    ++ph;
  };

  // ---- prologue: group 0 stages item 0 ----
  if (grp == 0) {
    load_input(0);
    store_input();
  }
  load_weights(decode(0));
  __syncthreads();
  if (grp == 1) {                                       // phase 0: stage item 1
    if (1 < count) {
      load_input(1);
      store_input();
    }
    phase_end();
  }
  for (int t = grp; t < count; t += 2) {
    compute(t);                                         // phase t
    phase_end();
    // phase t + 1: residual and next-item loads in flight while item t is finished
    if (has_res) res_issue(0);
    if (t + 2 < count) load_input(t + 2);
    if (has_res) {
      // the second residual half lands while the next input is staged
      finish(std::true_type{}, 0);
      res_issue(2);
      if (t + 2 < count) store_input();
      finish(std::true_type{}, 2);
    } else {
      finish(std::false_type{}, 0);
      finish(std::false_type{}, 2);
      if (t + 2 < count) store_input();
    }
    phase_end();
  }
  while (ph <= count) phase_end();
}

// packed[i][co][r][s][c] = c < ci ? w[i*co_n + co][c][r][s] : 0
template <typename T>
__global__ __launch_bounds__(256) void conv_pack_kernel(const T* __restrict__ w, T* __restrict__ out,
                                                        int64_t total, int ci, int ci32, int taps) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= total) return;
  const int c = static_cast<int>(e % ci32);
  const int64_t rest = e / ci32;                 // (i*co + co) * taps + tap
  const int tap = static_cast<int>(rest % taps);
  const int64_t oc = rest / taps;                // i*co + co
  out[e] = c < ci ? w[(oc * ci + c) * taps + tap] : from_f32<T>(0.f);
}

template <typename K>
int32_t launch_big_lds(K kernel, const ConvParams& p, dim3 grid, size_t lds, hipStream_t st) {
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess)
      return set_error(static_cast<int32_t>(e), "wc_conv2d: LDS of %zu bytes refused: %s", lds,
                       hipGetErrorString(e));
  }
  kernel<<<grid, kConvThreads, lds, st>>>(p);
  return check_launch("wc_conv2d");
}

constexpr size_t kConvLdsBudget = 152 * 1024;

inline int round32(int v) { return (v + 31) & ~31; }

// Tile / chunk plan; false if even the smallest tile does not fit in LDS.
template <typename T>
bool conv_plan(ConvParams& p) {
  constexpr int TPIX = 4 * ConvTraits<T>::kFM * 16;
  constexpr int PAD = ConvTraits<T>::kPad;
  p.ci32 = round32(p.ci);
  p.tc = p.wo < TPIX ? p.wo : TPIX;
  p.tr = TPIX / p.tc;
  if (p.tr > p.ho) p.tr = p.ho;
  for (;;) {
    p.ir = (p.tr - 1) * p.sh + (p.kh - 1) * p.dh + 1;
    p.ic = (p.tc - 1) * p.sw + (p.kw - 1) * p.dw + 1;
    const size_t epi = static_cast<size_t>(64) * (TPIX + 8) * sizeof(T);
    for (p.cc = p.ci32; p.cc >= 32; p.cc -= 32) {
      if (p.ci32 % p.cc) continue;
      const size_t in = static_cast<size_t>(p.ir) * p.ic * (p.cc + PAD) * sizeof(T);
      if ((in > epi ? in : epi) <= kConvLdsBudget) return true;
    }
    if (p.tr > 1) {
      p.tr = (p.tr + 1) / 2;
    } else if (p.tc > 16) {
      p.tc = (p.tc + 1) / 2;
    } else {
      return false;
    }
  }
}

// Tile plan of the fast kernel (256-pixel tiles, one LDS stage of 32
// channels, ideally <= 80 KB so two workgroups share a CU); false if it does
// not fit.
bool conv_fast_plan(ConvParams& p) {
  constexpr int TPIX = 256;
  const int taps = p.kh * p.kw;
  p.tc = p.wo < TPIX ? p.wo : TPIX;
  p.tr = TPIX / p.tc;
  if (p.tr > p.ho) p.tr = p.ho;
  const size_t epi = static_cast<size_t>(64) * (TPIX + 8) * sizeof(bf16);
  for (;;) {
    p.ir = p.tr + (p.kh - 1) * p.dh;
    p.ic = p.tc + (p.kw - 1) * p.dw;
    const size_t stage = (static_cast<size_t>(p.ir) * p.ic + static_cast<size_t>(taps) * 64) * kFPitch * sizeof(bf16);
    if (stage < epi) return false;                // the epilogue must fit in the stage buffer
    if (stage + 16 <= 80 * 1024) return true;
    if (p.tr > 1) p.tr = (p.tr + 1) / 2;
    else if (p.tc > 64) p.tc = (p.tc + 1) / 2;
    else return stage + 16 <= kConvLdsBudget;
  }
}

template <int KH, int KW, int CI, int W, typename PT>
int32_t conv_res_launch(ConvParams p, hipStream_t st) {
  using C = ResConv<KH, KW, CI, W>;
  const int64_t items = static_cast<int64_t>(p.n) * p.tiles_co * p.batch * cdiv(p.ho, C::TR);
  if (items >= 0x7fffffffll) return set_error(WC_ERR_LIMIT, "wc_conv2d: too many tiles");
  const int cus = device_cu_count();
  if (cus <= 0) return set_error(WC_ERR_ARG, "wc_conv2d: cannot query the CU count");
  const int grid = static_cast<int>(items < cus ? items : cus);
  const int per_wg = static_cast<int>(items / grid), extra = static_cast<int>(items % grid);
  auto kern = conv_res_kernel<KH, KW, CI, W, PT>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
  if (e != hipSuccess)
    return set_error(static_cast<int32_t>(e), "wc_conv2d: LDS of %d bytes refused: %s", C::LDS,
                     hipGetErrorString(e));
  kern<<<dim3(grid), dim3(512), C::LDS, st>>>(p, per_wg, extra);
  return check_launch("wc_conv2d");
}

// The (kh, kw, C_in, W) shapes the resident-weight kernel is instantiated for.
bool res_shape(int kh, int kw, int ci, int w) {
  return (kh == 3 && kw == 3 && ((ci == 64 && (w == 32 || w == 16)) || (ci == 32 && (w == 32 || w == 64)))) ||
         (kh == 1 && kw == 3 && (ci == 64 || ci == 32) && w == 256);
}

// True when the resident-weight kernel runs these sizes (bf16 'same' convolution, stride
// 1, C_in 32 / 64, C_out % 64 == 0, the vector alignments its loads and stores need).
bool conv_res_ok(const ConvParams& p) {
  const bool same = p.sh == 1 && p.sw == 1 && p.dh == 1 && p.dw == 1 && p.ph == p.kh / 2 && p.pw == p.kw / 2 &&
                    (p.kh % 2) == 1 && (p.kw % 2) == 1 && p.ho == p.h && p.wo == p.w;
  if (!same || p.co % 64 != 0 || !(p.ci == 32 || p.ci == 64) || !res_shape(p.kh, p.kw, p.ci, p.w)) return false;
  // one (model, batch row) block of x and of y / residual in bytes: a buffer descriptor's range
  if (static_cast<int64_t>(p.ci) * p.h * p.w * 2 >= 0x7fffffffll ||
      static_cast<int64_t>(p.co) * p.ho * p.wo * 2 >= 0x7fffffffll)
    return false;
  // 16-byte input and weight vectors, 8-byte output / residual vectors
  if (!aligned(p.x, 16) || (p.x_sn % 8) || (p.x_sb % 8) || !aligned(p.y, 8) || (p.y_sn % 4) || (p.y_sb % 4) ||
      !aligned(p.wn ? p.wn : p.wp, 16))
    return false;
  return !p.res || (aligned(p.res, 8) && (p.r_sn % 4) == 0 && (p.r_sb % 4) == 0);
}

// Launches the resident-weight kernel when conv_res_ok; returns 1 (nothing launched)
// otherwise.
int32_t conv_res_dispatch(ConvParams p, hipStream_t st) {
  if (!conv_res_ok(p)) return 1;
  p.tiles_co = p.co / 64;
  const bool pf = p.pdt == WC_F32;
#define WC_RES(KH, KW, CI, W)                                                                        \
  if (p.kh == KH && p.kw == KW && p.ci == CI && p.w == W)                                         \
    return pf ? conv_res_launch<KH, KW, CI, W, float>(p, st) : conv_res_launch<KH, KW, CI, W, bf16>(p, st);
  WC_RES(3, 3, 64, 32) WC_RES(3, 3, 64, 16) WC_RES(3, 3, 32, 32) WC_RES(3, 3, 32, 64)
  WC_RES(1, 3, 64, 256) WC_RES(1, 3, 32, 256)
#undef WC_RES
  return 1;
}

}  // namespace
}  // namespace wc

using namespace wc;

extern "C" int32_t wc_conv_pack_weights(const void* w, int64_t n, int64_t c_out, int64_t c_in, int64_t kh,
                                        int64_t kw, int32_t dtype, void* out, void* stream) {
  clear_error();
  WC_REQUIRE(n >= 0 && c_out >= 0 && c_in > 0 && kh > 0 && kw > 0, WC_ERR_SHAPE, "wc_conv_pack_weights: bad sizes");
  if (n == 0 || c_out == 0) return WC_OK;
  WC_REQUIRE(w && out, WC_ERR_NULL, "wc_conv_pack_weights: null pointer");
  // one thread per packed element, in a grid of at most 2^31 workgroups
  WC_REQUIRE(c_in < 0x7fffffe0ll && mul_sat({n, c_out, kh, kw, c_in + 31}) < (int64_t{1} << 39), WC_ERR_LIMIT,
             "wc_conv_pack_weights: sizes too large");
  const int ci32 = round32(static_cast<int>(c_in));
  const int64_t total = n * c_out * kh * kw * ci32;
  const dim3 grid(static_cast<uint32_t>(cdiv(total, 256)));
  hipStream_t st = as_stream(stream);
  if (dtype == WC_F32)
    conv_pack_kernel<float><<<grid, 256, 0, st>>>(static_cast<const float*>(w), static_cast<float*>(out), total,
                                                  (int)c_in, ci32, (int)(kh * kw));
  else if (dtype == WC_BF16)
    conv_pack_kernel<bf16><<<grid, 256, 0, st>>>(static_cast<const bf16*>(w), static_cast<bf16*>(out), total,
                                                 (int)c_in, ci32, (int)(kh * kw));
  else if (dtype == WC_F16)
    conv_pack_kernel<f16><<<grid, 256, 0, st>>>(static_cast<const f16*>(w), static_cast<f16*>(out), total,
                                                (int)c_in, ci32, (int)(kh * kw));
  else
    return set_error(WC_ERR_DTYPE, "wc_conv_pack_weights: unsupported dtype %s", dtype_name(dtype));
  return check_launch("wc_conv_pack_weights");
}

extern "C" int64_t wc_conv_packed_weight_elems(int64_t n, int64_t c_out, int64_t c_in, int64_t kh, int64_t kw) {
  if (n < 0 || c_out < 0 || c_in <= 0 || kh <= 0 || kw <= 0 || c_in >= 0x7fffffe0ll) return -1;
  const int64_t e = mul_sat({n, c_out, kh, kw, round32(static_cast<int>(c_in))});
  return e == INT64_MAX ? -1 : e;
}

extern "C" int32_t wc_conv2d_direct_weights(const wc_conv_args* a) {
  if (!a || a->dtype != WC_BF16 || !a->weight || a->n <= 0 || a->batch <= 0 || a->c_out <= 0 || a->h <= 0 ||
      a->w <= 0 || a->stride_h <= 0 || a->stride_w <= 0 || a->dil_h <= 0 || a->dil_w <= 0)
    return 0;
  if (!fits_i32({a->n, a->batch, a->c_in, a->c_out, a->h, a->w, a->kh, a->kw, a->stride_h, a->stride_w,
                 a->pad_h, a->pad_w, a->dil_h, a->dil_w, a->h_out, a->w_out}) ||
      mul_sat({a->c_in, a->h, a->w}) >= 0x7fffffffll || mul_sat({a->n, a->c_out}) >= 0x7fffffffll)
    return 0;
  ConvParams p = {};
  p.ci = (int)a->c_in;
  p.co = (int)a->c_out;
  p.h = (int)a->h;
  p.w = (int)a->w;
  p.kh = (int)a->kh;
  p.kw = (int)a->kw;
  p.sh = (int)a->stride_h;
  p.sw = (int)a->stride_w;
  p.ph = (int)a->pad_h;
  p.pw = (int)a->pad_w;
  p.dh = (int)a->dil_h;
  p.dw = (int)a->dil_w;
  p.ho = (int)a->h_out;
  p.wo = (int)a->w_out;
  p.x = a->x;
  p.x_sn = a->x_stride_n;
  p.x_sb = a->x_stride_b;
  p.wn = a->weight;
  p.res = a->residual;
  p.r_sn = a->r_stride_n;
  p.r_sb = a->r_stride_b;
  p.y = a->y;
  p.y_sn = a->y_stride_n;
  p.y_sb = a->y_stride_b;
  return conv_res_ok(p) ? 1 : 0;
}

extern "C" int32_t wc_conv2d(const wc_conv_args* a, void* stream) {
  clear_error();
  WC_REQUIRE(a != nullptr, WC_ERR_NULL, "wc_conv2d: null args");
  WC_REQUIRE(a->dtype == WC_F32 || a->dtype == WC_BF16 || a->dtype == WC_F16, WC_ERR_DTYPE,
             "wc_conv2d: unsupported dtype %s", dtype_name(a->dtype));
  WC_REQUIRE(a->param_dtype == WC_F32 || a->param_dtype == a->dtype, WC_ERR_DTYPE,
             "wc_conv2d: parameter dtype %s", dtype_name(a->param_dtype));
  WC_REQUIRE(a->n >= 0 && a->batch >= 0 && a->c_in > 0 && a->c_out >= 0 && a->h > 0 && a->w > 0 &&
                 a->kh > 0 && a->kw > 0 && a->stride_h > 0 && a->stride_w > 0 && a->pad_h >= 0 &&
                 a->pad_w >= 0 && a->dil_h > 0 && a->dil_w > 0,
             WC_ERR_SHAPE, "wc_conv2d: bad sizes");
  WC_REQUIRE(fits_i32({a->n, a->batch, a->c_in, a->c_out, a->h, a->w, a->kh, a->kw, a->stride_h, a->stride_w,
                       a->pad_h, a->pad_w, a->dil_h, a->dil_w}),
             WC_ERR_LIMIT, "wc_conv2d: sizes too large");
  const int64_t ho = (a->h + 2 * a->pad_h - a->dil_h * (a->kh - 1) - 1) / a->stride_h + 1;
  const int64_t wo = (a->w + 2 * a->pad_w - a->dil_w * (a->kw - 1) - 1) / a->stride_w + 1;
  WC_REQUIRE(ho == a->h_out && wo == a->w_out, WC_ERR_SHAPE,
             "wc_conv2d: output %lldx%lld does not match the geometry (%lldx%lld)", (long long)a->h_out,
             (long long)a->w_out, (long long)ho, (long long)wo);
  if (a->n == 0 || a->batch == 0 || a->c_out == 0 || ho <= 0 || wo <= 0) return WC_OK;
  WC_REQUIRE(a->x && a->y && (a->packed_weight || a->weight), WC_ERR_NULL, "wc_conv2d: null pointer");
  WC_REQUIRE(mul_sat({a->c_in, a->h, a->w}) < 0x7fffffffll && mul_sat({a->c_out, ho, wo}) < 0x7fffffffll &&
                 mul_sat({a->n, a->c_out}) < 0x7fffffffll,
             WC_ERR_LIMIT, "wc_conv2d: sizes too large");
  ConvParams p;
  p.n = (int)a->n;
  p.batch = (int)a->batch;
  p.ci = (int)a->c_in;
  p.co = (int)a->c_out;
  p.h = (int)a->h;
  p.w = (int)a->w;
  p.kh = (int)a->kh;
  p.kw = (int)a->kw;
  p.sh = (int)a->stride_h;
  p.sw = (int)a->stride_w;
  p.ph = (int)a->pad_h;
  p.pw = (int)a->pad_w;
  p.dh = (int)a->dil_h;
  p.dw = (int)a->dil_w;
  p.ho = (int)ho;
  p.wo = (int)wo;
  p.act = a->act;
  p.x = a->x;
  p.x_sn = a->x_stride_n;
  p.x_sb = a->x_stride_b;
  p.wp = a->packed_weight;
  p.wn = a->packed_weight ? nullptr : a->weight;
  p.bias = a->bias;
  p.bn_w = a->bn_weight;
  p.bn_b = a->bn_bias;
  p.bn_mean = a->bn_mean;
  p.bn_var = a->bn_var;
  p.bn_eps = a->bn_eps;
  p.pdt = a->param_dtype;
  WC_REQUIRE(!p.bn_mean || p.bn_var, WC_ERR_NULL, "wc_conv2d: BN mean without variance");
  p.res = a->residual;
  p.r_sn = a->r_stride_n;
  p.r_sb = a->r_stride_b;
  p.y = a->y;
  p.y_sn = a->y_stride_n;
  p.y_sb = a->y_stride_b;
  p.kd = p.sd = p.dd = p.d = p.dout = 1;
  p.pd = 0;
  p.x_cs = static_cast<int64_t>(p.h) * p.w;
  p.y_cs = static_cast<int64_t>(p.ho) * p.wo;
  const bool f32 = a->dtype == WC_F32;
  const bool f16m = a->dtype == WC_F16;              // fp16: the general kernel only
  if (!(f32 ? conv_plan<float>(p) : conv_plan<bf16>(p)))
    return set_error(WC_ERR_LIMIT, "wc_conv2d: tile does not fit in LDS");
  p.fd_plane = make_fastdiv(static_cast<uint32_t>(p.ir * p.ic));
  p.fd_ic = make_fastdiv(static_cast<uint32_t>(p.ic));
  p.tiles_r = static_cast<int>(cdiv(p.ho, p.tr));
  p.tiles_c = static_cast<int>(cdiv(p.wo, p.tc));
  p.tiles_co = static_cast<int>(cdiv(p.co, 64));
  const int es = f32 ? 4 : 2;
  const int ve = 16 / es;
  const bool yal = aligned(p.y, 16) && ubytes(p.y_sn, es) % 16 == 0 && ubytes(p.y_sb, es) % 16 == 0;
  const bool ral = !p.res || (aligned(p.res, 16) && ubytes(p.r_sn, es) % 16 == 0 && ubytes(p.r_sb, es) % 16 == 0);
  p.vec_out = (yal && ral && p.tc % ve == 0 && p.wo % ve == 0) ? 1 : 0;
  if (p.wn) {
    // the filter bank itself: only the resident-weight kernel reads that layout
    WC_REQUIRE(!f32 && !f16m && conv_res_ok(p), WC_ERR_ARG,
               "wc_conv2d: these sizes need packed weights (wc_conv_pack_weights); "
               "wc_conv2d_direct_weights tells when the filter bank itself will do");
    return conv_res_dispatch(p, as_stream(stream));
  }
  WC_REQUIRE(aligned(p.wp, 16), WC_ERR_ALIGN, "wc_conv2d: packed weights not 16-byte aligned");
  const int64_t nblk = static_cast<int64_t>(p.n) * p.batch * p.tiles_r * p.tiles_c * p.tiles_co;
  WC_REQUIRE(nblk < 0x7fffffffll, WC_ERR_LIMIT, "wc_conv2d: too many tiles");
  p.remap = (nblk % 8 == 0) ? 1 : 0;
  const size_t in = static_cast<size_t>(p.ir) * p.ic * (p.cc + (f32 ? 4 : 8)) * es;
  const size_t epi = static_cast<size_t>(64) * (4 * (f32 ? 4 : 8) * 16 + 8) * es;
  const size_t lds = in > epi ? in : epi;
  hipStream_t st = as_stream(stream);
  // resident-weight path: bf16 "same" convolution, stride 1, C_in 32 / 64, C_out % 64 == 0
  if (!f32 && !f16m) {
    const int32_t rc = conv_res_dispatch(p, st);
    if (rc != 1) return rc;
  }
  // fast path: weights and input chunk both staged in LDS (bf16, stride 1, W % 8 == 0)
  if (!f32 && !f16m && p.sh == 1 && p.sw == 1 && p.kh * p.kw <= kFastTaps && p.w % 8 == 0 && aligned(p.x, 16) &&
      ubytes(p.x_sn, es) % 16 == 0 && ubytes(p.x_sb, es) % 16 == 0 && (static_cast<int64_t>(p.h) * p.w * es) % 16 == 0) {
    ConvParams q = p;
    if (conv_fast_plan(q)) {
      q.tiles_r = static_cast<int>(cdiv(q.ho, q.tr));
      q.tiles_c = static_cast<int>(cdiv(q.wo, q.tc));
      q.vec_out = (yal && ral && q.tc % ve == 0 && q.wo % ve == 0) ? 1 : 0;
      const int64_t fblk = static_cast<int64_t>(q.n) * q.batch * q.tiles_r * q.tiles_c * q.tiles_co;
      WC_REQUIRE(fblk < 0x7fffffffll, WC_ERR_LIMIT, "wc_conv2d: too many tiles");
      q.remap = (fblk % 8 == 0) ? 1 : 0;
      // one item per workgroup, one LDS stage (two workgroups share a CU, so one
      // workgroup's staging and epilogue overlap the other's MFMAs)
      const size_t stage = (static_cast<size_t>(q.ir) * q.ic + static_cast<size_t>(q.kh) * q.kw * 64) * kFPitch * es;
      const size_t flds = stage + 16;
      const bool k9 = q.kh * q.kw == 9;
      auto kern = q.pdt == WC_F32 ? (k9 ? conv_persist_kernel<float, false, 9> : conv_persist_kernel<float, false, 0>)
                                  : (k9 ? conv_persist_kernel<bf16, false, 9> : conv_persist_kernel<bf16, false, 0>);
      if (flds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(flds));
        if (e != hipSuccess)
          return set_error(static_cast<int32_t>(e), "wc_conv2d: LDS of %zu bytes refused: %s", flds,
                           hipGetErrorString(e));
      }
      kern<<<dim3(static_cast<uint32_t>(fblk)), kConvThreads, flds, st>>>(q, 1, 0);
      return check_launch("wc_conv2d");
    }
  }
  const dim3 grid(static_cast<uint32_t>(nblk));
  if (f32) return launch_big_lds(conv_kernel<float>, p, grid, lds, st);
  if (f16m) return launch_big_lds(conv_kernel<f16>, p, grid, lds, st);
  return launch_big_lds(conv_kernel<bf16>, p, grid, lds, st);
}

extern "C" int32_t wc_conv3d(const wc_conv3d_args* a, void* stream) {
  clear_error();
  WC_REQUIRE(a != nullptr, WC_ERR_NULL, "wc_conv3d: null args");
  WC_REQUIRE(a->dtype == WC_F32 || a->dtype == WC_BF16 || a->dtype == WC_F16, WC_ERR_DTYPE,
             "wc_conv3d: unsupported dtype %s", dtype_name(a->dtype));
  WC_REQUIRE(a->param_dtype == WC_F32 || a->param_dtype == a->dtype, WC_ERR_DTYPE,
             "wc_conv3d: parameter dtype %s", dtype_name(a->param_dtype));
  WC_REQUIRE(a->act == WC_ACT_NONE || a->act == WC_ACT_RELU, WC_ERR_ARG, "wc_conv3d: bad act %d", a->act);
  WC_REQUIRE(a->n >= 0 && a->batch >= 0 && a->c_in > 0 && a->c_out >= 0 && a->d > 0 && a->h > 0 && a->w > 0 &&
                 a->kd > 0 && a->kh > 0 && a->kw > 0 && a->stride_d > 0 && a->stride_h > 0 && a->stride_w > 0 &&
                 a->pad_d >= 0 && a->pad_h >= 0 && a->pad_w >= 0 && a->dil_d > 0 && a->dil_h > 0 && a->dil_w > 0,
             WC_ERR_SHAPE, "wc_conv3d: bad sizes");
  WC_REQUIRE(fits_i32({a->n, a->batch, a->c_in, a->c_out, a->d, a->h, a->w, a->kd, a->kh, a->kw, a->stride_d,
                       a->stride_h, a->stride_w, a->pad_d, a->pad_h, a->pad_w, a->dil_d, a->dil_h, a->dil_w}),
             WC_ERR_LIMIT, "wc_conv3d: sizes too large");
  const int64_t dout = (a->d + 2 * a->pad_d - a->dil_d * (a->kd - 1) - 1) / a->stride_d + 1;
  const int64_t ho = (a->h + 2 * a->pad_h - a->dil_h * (a->kh - 1) - 1) / a->stride_h + 1;
  const int64_t wo = (a->w + 2 * a->pad_w - a->dil_w * (a->kw - 1) - 1) / a->stride_w + 1;
  WC_REQUIRE(dout == a->d_out && ho == a->h_out && wo == a->w_out, WC_ERR_SHAPE,
             "wc_conv3d: output %lldx%lldx%lld does not match the geometry (%lldx%lldx%lld)", (long long)a->d_out,
             (long long)a->h_out, (long long)a->w_out, (long long)dout, (long long)ho, (long long)wo);
  if (a->n == 0 || a->batch == 0 || a->c_out == 0 || dout <= 0 || ho <= 0 || wo <= 0) return WC_OK;
  WC_REQUIRE(a->x && a->packed_weight && a->y, WC_ERR_NULL, "wc_conv3d: null pointer");
  WC_REQUIRE(mul_sat({a->c_in, a->d, a->h, a->w}) < 0x7fffffffll &&
                 mul_sat({a->c_out, dout, ho, wo}) < 0x7fffffffll && mul_sat({a->n, a->c_out}) < 0x7fffffffll &&
                 mul_sat({a->kd, a->kh, a->kw}) < 0x10000,
             WC_ERR_LIMIT, "wc_conv3d: sizes too large");
  ConvParams p;
  p.n = (int)a->n;
  p.batch = (int)a->batch;
  p.ci = (int)a->c_in;
  p.co = (int)a->c_out;
  p.h = (int)a->h;
  p.w = (int)a->w;
  p.kh = (int)a->kh;
  p.kw = (int)a->kw;
  p.sh = (int)a->stride_h;
  p.sw = (int)a->stride_w;
  p.ph = (int)a->pad_h;
  p.pw = (int)a->pad_w;
  p.dh = (int)a->dil_h;
  p.dw = (int)a->dil_w;
  p.ho = (int)ho;
  p.wo = (int)wo;
  p.kd = (int)a->kd;
  p.sd = (int)a->stride_d;
  p.pd = (int)a->pad_d;
  p.dd = (int)a->dil_d;
  p.d = (int)a->d;
  p.dout = (int)dout;
  p.x_cs = a->d * a->h * a->w;
  p.y_cs = dout * ho * wo;
  p.act = a->act;
  p.x = a->x;
  p.x_sn = a->x_stride_n;
  p.x_sb = a->x_stride_b;
  p.wp = a->packed_weight;
  p.wn = nullptr;
  p.bias = a->bias;
  p.bn_w = p.bn_b = p.bn_mean = p.bn_var = nullptr;
  p.bn_eps = 0.f;
  p.pdt = a->param_dtype;
  p.res = nullptr;
  p.r_sn = p.r_sb = 0;
  p.y = a->y;
  p.y_sn = a->y_stride_n;
  p.y_sb = a->y_stride_b;
  const bool f32 = a->dtype == WC_F32;
  const bool f16m = a->dtype == WC_F16;              // fp16: the general kernel only
  if (!(f32 ? conv_plan<float>(p) : conv_plan<bf16>(p)))
    return set_error(WC_ERR_LIMIT, "wc_conv3d: tile does not fit in LDS");
  p.fd_plane = make_fastdiv(static_cast<uint32_t>(p.ir * p.ic));
  p.fd_ic = make_fastdiv(static_cast<uint32_t>(p.ic));
  p.tiles_r = static_cast<int>(cdiv(p.ho, p.tr));
  p.tiles_c = static_cast<int>(cdiv(p.wo, p.tc));
  p.tiles_co = static_cast<int>(cdiv(p.co, 64));
  const int es = f32 ? 4 : 2;
  const int ve = 16 / es;
  const bool yal = aligned(p.y, 16) && ubytes(p.y_sn, es) % 16 == 0 && ubytes(p.y_sb, es) % 16 == 0 &&
                   ubytes(p.y_cs, es) % 16 == 0 && (static_cast<int64_t>(p.ho) * p.wo * es) % 16 == 0;
  p.vec_out = (yal && p.tc % ve == 0 && p.wo % ve == 0) ? 1 : 0;
  WC_REQUIRE(aligned(p.wp, 16), WC_ERR_ALIGN, "wc_conv3d: packed weights not 16-byte aligned");
  const int64_t nblk = static_cast<int64_t>(p.n) * p.batch * p.dout * p.tiles_r * p.tiles_c * p.tiles_co;
  WC_REQUIRE(nblk < 0x7fffffffll, WC_ERR_LIMIT, "wc_conv3d: too many tiles");
  p.remap = (nblk % 8 == 0) ? 1 : 0;
  const size_t in = static_cast<size_t>(p.ir) * p.ic * (p.cc + (f32 ? 4 : 8)) * es;
  const size_t epi = static_cast<size_t>(64) * (4 * (f32 ? 4 : 8) * 16 + 8) * es;
  const size_t lds = in > epi ? in : epi;
  const dim3 grid(static_cast<uint32_t>(nblk));
  hipStream_t st = as_stream(stream);
  if (f32) return launch_big_lds(conv_kernel<float>, p, grid, lds, st);
  if (f16m) return launch_big_lds(conv_kernel<f16>, p, grid, lds, st);
  return launch_big_lds(conv_kernel<bf16>, p, grid, lds, st);
}
