// Fused multi-head attention (softmax(Q K^T * scale) V per (model, batch, head))
// on MFMA with an online (flash-style) softmax over key tiles.
//
// Layout: Q, K, V, O are read / written in place in the [N*B, S, heads*Dh]
// layout the projection GEMMs produce (head h = columns [h*Dh, (h+1)*Dh)), so no
// head-major copies are made.
//
// Per workgroup: one (model*batch, head) pair and a tile of 128 queries, four
// waves of 32 queries each.  For every tile of 64 keys:
//   S^T = K Q^T          (MFMA; the output layout puts 4 consecutive keys of
//                         one query in each lane)
//   online softmax       column-wise over keys: running max m and sum l per query
//   O^T += V^T P^T       (MFMA; P^T is consumed straight from the S^T registers:
//                         the 32-key reduction step takes keys {4g..4g+3,
//                         16+4g..16+4g+3} from lane group g, and V^T is read from
//                         LDS in that same key order, so P never goes through LDS)
// K tiles are staged in LDS row-major, V tiles transposed (V^T [Dh][keys]); the
// next tile is fetched into registers while the current one is processed.
// Scores are scaled by log2(e)/sqrt(Dh) so the exponentials are v_exp_f32 (2^x).
#include "wc_common.h"

#include <type_traits>

namespace wc {
namespace {

struct AttnParams {
  int nb, heads, sq, skv, causal, q_tiles;
  float scale_log2;
  const void* q;
  int64_t q_sb, q_ss;
  const void* k;
  int64_t k_sb, k_ss;
  const void* v;
  int64_t v_sb, v_ss;
  void* o;
  int64_t o_sb, o_ss;
  // additive fp32 mask, element (nb, head, query, key) at nb*m_sb + head*m_sh + query*m_sq + key
  // (general kernel only; NULL = none)
  const float* mask;
  int64_t m_sb, m_sh, m_sq;
};

constexpr int kAttnThreads = 256;
constexpr int kBQ = 128;   // queries per workgroup (32 per wave)
constexpr int kBK = 64;    // keys per tile

__device__ __forceinline__ float xor_max(float v, int m) { return fmaxf(v, __shfl_xor(v, m, 64)); }
__device__ __forceinline__ float xor_sum(float v, int m) { return v + __shfl_xor(v, m, 64); }

template <typename T, int DH>
__global__ __launch_bounds__(kAttnThreads) void attn_kernel(AttnParams p) {
  constexpr bool BF = sizeof(T) == 2;
  constexpr int DHP = DH < 32 ? 32 : DH;       // head dim padded to the 32-wide S^T k-step
  constexpr int KP = DHP + (BF ? 8 : 4);       // K tile pitch (elements)
  constexpr int VP = kBK + (BF ? 8 : 4);       // V^T tile pitch (elements)
  constexpr int DT = DH / 16;                  // 16-row tiles of O^T
  constexpr int NKS = DHP / 32;                // 32-wide head-dim steps of S^T = K Q^T
  extern __shared__ float4 smem4[];
  T* const ks0 = reinterpret_cast<T*>(smem4);   // [2][kBK * KP]  K tiles
  T* const vt0 = ks0 + 2 * kBK * KP;            // [2][DH * VP]   V^T tiles

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int fr = lane & 15, g = lane >> 4;
  const int qt = blockIdx.x % p.q_tiles;
  const int bh = blockIdx.x / p.q_tiles;
  const int nb = bh / p.heads, h = bh - (bh / p.heads) * p.heads;
  const T* qb = static_cast<const T*>(p.q) + nb * p.q_sb + h * DH;
  const T* kb = static_cast<const T*>(p.k) + nb * p.k_sb + h * DH;
  const T* vb = static_cast<const T*>(p.v) + nb * p.v_sb + h * DH;
  T* ob = static_cast<T*>(p.o) + nb * p.o_sb + h * DH;
  const int q0 = qt * kBQ + wave * 32;           // first query of this wave

  // ---- Q^T fragments (B operand of S^T = K Q^T), kept in registers ----
  // lane supplies Q[q = q0 + nt*16 + fr][d = s*32 + g*8 .. +8] (fp32: two 16-byte halves)
  uint4 qf[2][NKS][2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int q = q0 + nt * 16 + fr;
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      const T* src = qb + q * p.q_ss + s * 32 + g * 8;
      const bool ok = q < p.sq && s * 32 + g * 8 < DH;   // head-dim padding reads as zero
      qf[nt][s][0] = ok ? *reinterpret_cast<const uint4*>(src) : make_uint4(0, 0, 0, 0);
      qf[nt][s][1] = (!BF && ok) ? *reinterpret_cast<const uint4*>(src + (BF ? 0 : 4)) : make_uint4(0, 0, 0, 0);
    }
  }

  // ---- staging of one K / V tile: each thread moves one 16-byte row piece of each ----
  constexpr int VE = 16 / sizeof(T);
  constexpr int PIECES = kBK * DH / VE;          // 16-byte pieces per tile
  uint4 kreg[(PIECES + kAttnThreads - 1) / kAttnThreads], vreg[(PIECES + kAttnThreads - 1) / kAttnThreads];
  constexpr int PPT = (PIECES + kAttnThreads - 1) / kAttnThreads;
  auto fetch = [&](int k0) {
#pragma unroll
    for (int u = 0; u < PPT; ++u) {
      const int e = tid + u * kAttnThreads;
      const int key = e / (DH / VE), c = (e - key * (DH / VE)) * VE;
      const bool ok = e < PIECES && k0 + key < p.skv;
      kreg[u] = ok ? *reinterpret_cast<const uint4*>(kb + (k0 + key) * p.k_ss + c) : make_uint4(0, 0, 0, 0);
      vreg[u] = ok ? *reinterpret_cast<const uint4*>(vb + (k0 + key) * p.v_ss + c) : make_uint4(0, 0, 0, 0);
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int u = 0; u < PPT; ++u) {
      const int e = tid + u * kAttnThreads;
      if (e >= PIECES) continue;
      const int key = e / (DH / VE), c = (e - key * (DH / VE)) * VE;
      *reinterpret_cast<uint4*>(&ks0[buf * kBK * KP + key * KP + c]) = kreg[u];
      const T* vv = reinterpret_cast<const T*>(&vreg[u]);
#pragma unroll
      for (int q = 0; q < VE; ++q) vt0[buf * DH * VP + (c + q) * VP + key] = vv[q];
    }
  };

  f32x4 acc_o[DT][2];
#pragma unroll
  for (int i = 0; i < DT; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc_o[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};

  int kend = p.skv;
  if (p.causal) {
    const int qlast = qt * kBQ + kBQ - 1;
    kend = qlast + 1 < p.skv ? qlast + 1 : p.skv;
  }
  const int ntiles = (kend + kBK - 1) / kBK;
  if (DHP != DH) {
    // zero the padded head-dim columns of both K buffers once (stash never writes them)
    for (int e = tid; e < 2 * kBK * (DHP - DH); e += kAttnThreads) {
      const int row = e / (DHP - DH), c = DH + (e - row * (DHP - DH));
      ks0[row * KP + c] = from_f32<T>(0.f);
    }
  }
  fetch(0);
  stash(0);
  __syncthreads();

  for (int kt = 0; kt < ntiles; ++kt) {
    const int buf = kt & 1;
    const int k0 = kt * kBK;
    if (kt + 1 < ntiles) fetch(k0 + kBK);
    const T* kt_s = ks0 + buf * kBK * KP;
    const T* vt_s = vt0 + buf * DH * VP;

    // ---- S^T = K Q^T : [64 keys x 32 queries] per wave ----
    f32x4 sacc[4][2];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) sacc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const T* krow = kt_s + (mt * 16 + fr) * KP + g * 8;
#pragma unroll
      for (int s = 0; s < NKS; ++s) {
        if constexpr (BF) {
          const bf16x8 a = *reinterpret_cast<const bf16x8*>(krow + s * 32);
#pragma unroll
          for (int nt = 0; nt < 2; ++nt)
            sacc[mt][nt] = mma16<T>(a, *reinterpret_cast<const bf16x8*>(&qf[nt][s][0]), sacc[mt][nt]);
        } else {
          const f32x4 a0 = *reinterpret_cast<const f32x4*>(krow + s * 32);
          const f32x4 a1 = *reinterpret_cast<const f32x4*>(krow + s * 32 + 4);
#pragma unroll
          for (int nt = 0; nt < 2; ++nt) {
            const f32x4 b0 = *reinterpret_cast<const f32x4*>(&qf[nt][s][0]);
            const f32x4 b1 = *reinterpret_cast<const f32x4*>(&qf[nt][s][1]);
#pragma unroll
            for (int j = 0; j < 4; ++j)
              sacc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[j], b0[j], sacc[mt][nt], 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 4; ++j)
              sacc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1[j], b1[j], sacc[mt][nt], 0, 0, 0);
          }
        }
      }
    }

    // ---- online softmax over keys (rows of S^T), per query column ----
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int q = q0 + nt * 16 + fr;
      const float* mrow = (p.mask && q < p.sq) ? p.mask + nb * p.m_sb + h * p.m_sh + q * p.m_sq : nullptr;
      float tmax = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int key = k0 + mt * 16 + g * 4 + e;
          float sv = sacc[mt][nt][e] * p.scale_log2;
          if (key >= p.skv || (p.causal && key > q))
            sv = -INFINITY;
          else if (mrow)
            sv += mrow[key] * 1.4426950408889634f;        // natural-log mask -> the exp2 domain
          sacc[mt][nt][e] = sv;
          tmax = fmaxf(tmax, sv);
        }
      tmax = xor_max(xor_max(tmax, 16), 32);
      const float m_new = fmaxf(m_run[nt], tmax);
      // rows with no valid key so far keep m = -inf; use 0 as the exponent base then
      const float base = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run[nt] - base);
      float tsum = 0.f;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float pv = __builtin_amdgcn_exp2f(sacc[mt][nt][e] - base);
          sacc[mt][nt][e] = pv;
          tsum += pv;
        }
      tsum = xor_sum(xor_sum(tsum, 16), 32);
      l_run[nt] = l_run[nt] * alpha + tsum;
      m_run[nt] = m_new;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc_o[dt][nt] *= alpha;
    }

    // ---- O^T += V^T P^T ----
    if constexpr (BF) {
#pragma unroll
      for (int s = 0; s < 2; ++s) {           // 32-key steps
        bf16x8 bp[2];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            // P in the operand type, carried as raw 16-bit lanes
            bp[nt][e] = __builtin_bit_cast(bf16, static_cast<T>(sacc[2 * s][nt][e]));
            bp[nt][4 + e] = __builtin_bit_cast(bf16, static_cast<T>(sacc[2 * s + 1][nt][e]));
          }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const T* vrow = vt_s + (dt * 16 + fr) * VP + s * 32 + g * 4;
          bf16x8 a;
          const bf16x4 lo = *reinterpret_cast<const bf16x4*>(vrow);
          const bf16x4 hi = *reinterpret_cast<const bf16x4*>(vrow + 16);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            a[e] = lo[e];
            a[4 + e] = hi[e];
          }
#pragma unroll
          for (int nt = 0; nt < 2; ++nt)
            acc_o[dt][nt] = mma16<T>(a, bp[nt], acc_o[dt][nt]);
        }
      }
    } else {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)          // 16-key tiles, 4 k-slots each
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const f32x4 a = *reinterpret_cast<const f32x4*>(vt_s + (dt * 16 + fr) * VP + mt * 16 + g * 4);
#pragma unroll
          for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              acc_o[dt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], sacc[mt][nt][j], acc_o[dt][nt], 0, 0, 0);
        }
    }

    if (kt + 1 < ntiles) {
      // buffer buf^1 was last read in the previous iteration, before its closing barrier
      stash(buf ^ 1);
      __syncthreads();
    }
  }

  // ---- O = (O^T / l)^T : lane holds O[q][d = dt*16 + g*4 + e] ----
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int q = q0 + nt * 16 + fr;
    if (q >= p.sq) continue;
    const float inv = l_run[nt] > 0.f ? 1.0f / l_run[nt] : 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      T* dst = ob + q * p.o_ss + dt * 16 + g * 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) dst[e] = from_f32<T>(acc_o[dt][nt][e] * inv);
    }
  }
}

// ---------------------------------------------------------------------------
// Resident-KV kernel (bf16, head dim 32 or 64, K and V of one head fit in LDS).
// One workgroup per (model*batch, head, tile of W*64 queries).  K (row-major,
// rows padded by 16 bytes) and V^T ([dh][key], rows padded by 8 bytes) of every
// key are staged in LDS once, so the key loop has no barriers.  Each wave owns
// 64 queries as two 32-query blocks and walks the keys in blocks of 32 with
// v_mfma_f32_32x32x16_bf16:
//   S^T = K Q^T      lane l holds query l%32 and 16 of the block's 32 keys
//                    (keys 8 (r/4) + 4 (l/32) + r%4 in register r)
//   softmax          block max in-lane over 16 keys, then across the lane
//                    halves with v_permlane32_swap (no LDS); the running max
//                    only moves when a block exceeds it by 2^8 (P <= 2^8 keeps
//                    fp32 sums exact enough), so most blocks skip the rescale
//   O^T += V^T P^T   P^T is the S^T register block itself: k-step j takes
//                    registers 8j..8j+7, i.e. keys 16j + 8 (s/4) + 4 (l/32) + s%4,
//                    and V^T is read from LDS in that key order (two 8-byte reads)
// Scores are scaled by log2(e)/sqrt(Dh) inside the exp2 argument (one FMA).
// ---------------------------------------------------------------------------
constexpr float kLazyRescale = 8.0f;
constexpr bf16x2 kOnes2 = {bf16(1.0f), bf16(1.0f)};

// (v of this lane, v of lane l ^ 32) via v_permlane32_swap on an opaque copy:
// the compiler folds the intrinsic when both operands are the same value, so
// the exchange is written out, with the wait states around the swap.
__device__ __forceinline__ void half_swap(float v, float& mine, float& other) {
  float a = v, b;
  asm volatile(
      "s_nop 1\n\t"
      "v_mov_b32 %1, %0\n\t"
      "s_nop 1\n\t"
      "v_permlane32_swap_b32 %0, %1\n\t"
      "s_nop 1"
      : "+v"(a), "=&v"(b));
  // a = {v[0:31], v[0:31]}, b = {v[32:63], v[32:63]}
  mine = v;
  other = (threadIdx.x & 32) ? a : b;
}
__device__ __forceinline__ float other_half_max(float v) {
  float m, o;
  half_swap(v, m, o);
  return fmaxf(m, o);
}
__device__ __forceinline__ float other_half_sum(float v) {
  float m, o;
  half_swap(v, m, o);
  return m + o;
}

template <int DH>
constexpr int res_kpitch() { return DH + 8; }      // K row pitch (bf16 elements)

inline size_t res_lds_bytes(int dh, int skvp) {
  return (static_cast<size_t>(skvp) * (dh + 8) + static_cast<size_t>(dh) * (skvp + 4)) * sizeof(bf16);
}

template <int DH, int W, bool CAUSAL>
__global__ __launch_bounds__(W * 64) void attn_res_kernel(AttnParams p, int skvp) {
  constexpr int KP = res_kpitch<DH>();
  constexpr int NKS = DH / 16;                       // 16-dim k-steps of S^T = K Q^T
  constexpr int DT = DH / 32;                        // 32-row tiles of O^T
  const int VTP = skvp + 4;                          // V^T row pitch (bf16 elements)
  extern __shared__ float4 smem4[];
  bf16* const ksm = reinterpret_cast<bf16*>(smem4);  // [skvp][KP]
  bf16* const vts = ksm + static_cast<int64_t>(skvp) * KP;   // [DH][VTP]

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, hf = lane >> 5;
  // Workgroups are dispatched round-robin over the 8 XCDs; XCD x takes the contiguous
  // range [x G / 8, (x + 1) G / 8) of (batch, head, query tile) ids, so the heads of one
  // row, whose 64-byte slices share cache lines, are read through one L2.
  const int G = gridDim.x;
  const int bid = (G & 7) == 0 ? (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  const int qt = bid % p.q_tiles;
  const int bh = bid / p.q_tiles;
  const int nb = bh / p.heads, h = bh - (bh / p.heads) * p.heads;
  const bf16* qb = static_cast<const bf16*>(p.q) + nb * p.q_sb + h * DH;
  const bf16* kb = static_cast<const bf16*>(p.k) + nb * p.k_sb + h * DH;
  const bf16* vb = static_cast<const bf16*>(p.v) + nb * p.v_sb + h * DH;
  bf16* ob = static_cast<bf16*>(p.o) + nb * p.o_sb + h * DH;

  // ---- stage K and V^T of all keys (keys >= skv read as zero) ----
  {
    constexpr int CPR = DH / 8;                      // 16-byte chunks per row
    constexpr int U = 4;                             // chunks per thread in flight
    const int total = skvp * CPR;
    for (int e0 = tid; e0 < total; e0 += U * W * 64) {
      uint4 kv[U], vv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int e = e0 + u * W * 64;
        const int key = e / CPR, c = (e - (e / CPR) * CPR) * 8;
        const bool ok = e < total && key < p.skv;
        kv[u] = ok ? *reinterpret_cast<const uint4*>(kb + static_cast<int64_t>(key) * p.k_ss + c) : make_uint4(0, 0, 0, 0);
        vv[u] = ok ? *reinterpret_cast<const uint4*>(vb + static_cast<int64_t>(key) * p.v_ss + c) : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int e = e0 + u * W * 64;
        if (e >= total) continue;
        const int key = e / CPR, c = (e - (e / CPR) * CPR) * 8;
        *reinterpret_cast<uint4*>(ksm + key * KP + c) = kv[u];
        const bf16* v8 = reinterpret_cast<const bf16*>(&vv[u]);
#pragma unroll
        for (int i = 0; i < 8; ++i) vts[(c + i) * VTP + key] = v8[i];
      }
    }
  }

  // ---- this wave's queries and their Q^T fragments (B operand of S^T) ----
  // first query rows of the wave's two 32-query blocks: blocks wave and 2W - 1 - wave of
  // the tile's 2W, so that under a causal mask every wave has the same number of key
  // blocks to process (a block is skipped for the query block it lies wholly after)
  const int qt0 = qt * (W * 64);
  const int qrow[2] = {qt0 + wave * 32, qt0 + (2 * W - 1 - wave) * 32};
  bf16x8 qf[2][NKS];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    int q = qrow[b] + l32;
    q = q < p.sq ? q : p.sq - 1;
#pragma unroll
    for (int k = 0; k < NKS; ++k)
      qf[b][k] = *reinterpret_cast<const bf16x8*>(qb + static_cast<int64_t>(q) * p.q_ss + 16 * k + 8 * hf);
  }
  // Q^T pre-scaled by scale * log2(e) (rounded back to bf16), so the MFMAs produce the
  // exponent of exp2 directly, and one more k-step adds the row's running base: K is
  // extended by a column of ones (kone: A operand, k = 0 of the lanes < 32) and Q^T by
  // the row of -base (qneg[b]: B operand, k = 0 of lane = query < 32).  The softmax
  // then needs one v_exp per score and no multiply-add.
  const float c = p.scale_log2;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int k = 0; k < NKS; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[b][k][e] = static_cast<bf16>(static_cast<float>(qf[b][k][e]) * c);
  bf16x8 kone, qneg[2];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    kone[e] = static_cast<bf16>(e == 0 && hf == 0 ? 1.0f : 0.0f);
    qneg[0][e] = static_cast<bf16>(0.0f);
    qneg[1][e] = static_cast<bf16>(0.0f);
  }
  __syncthreads();

  f32x16 oacc[2][DT];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int e = 0; e < 16; ++e) oacc[b][d][e] = 0.f;
  // base[b]: the bf16 value subtracted from this row's exponents (0 until the first block sets it)
  float base[2] = {0.f, 0.f}, lrun[2] = {0.f, 0.f};
  int nkb = skvp / 32;
  if (CAUSAL) {
    const int qmax = qrow[1] + 31;                  // qrow[1] >= qrow[0]
    const int last = (qmax < p.sq ? qmax : p.sq - 1) / 32 + 1;
    nkb = last < nkb ? last : nkb;
  }
  // one 32-key block: both query blocks' scores first (their MFMA latency hides
  // behind the first block's softmax), then per query block softmax and P V
  auto key_block = [&](int kbk, auto mask_tag, bool first) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const int key0 = kbk * 32;
    bf16x8 kf[NKS];
#pragma unroll
    for (int k = 0; k < NKS; ++k)
      kf[k] = *reinterpret_cast<const bf16x8*>(ksm + (key0 + l32) * KP + 16 * k + 8 * hf);
    bf16x8 vf[DT][2];
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const bf16* vr = vts + (d * 32 + l32) * VTP + key0 + 16 * j + 4 * hf;
        const bf16x4 lo = *reinterpret_cast<const bf16x4*>(vr);
        const bf16x4 hi = *reinterpret_cast<const bf16x4*>(vr + 8);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vf[d][j][e] = lo[e];
          vf[d][j][4 + e] = hi[e];
        }
      }
    f32x16 s[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      if (CAUSAL && key0 > qrow[b] + 31) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) s[b][e] = 0.f;
#pragma unroll
      for (int k = 0; k < NKS; ++k) s[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[k], qf[b][k], s[b], 0, 0, 0);
      s[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kone, qneg[b], s[b], 0, 0, 0);
    }
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      if (CAUSAL && key0 > qrow[b] + 31) continue;
      if constexpr (MASK) {
        const int q = qrow[b] + l32;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = key0 + (r >> 2) * 8 + 4 * hf + (r & 3);
          if (key >= p.skv || (CAUSAL && key > q)) s[b][r] = -INFINITY;
        }
      }
      // tree reductions keep the dependency chains short
      const float m0 = __builtin_fmaxf(__builtin_fmaxf(s[b][0], s[b][1]), s[b][2]);
      const float m1 = __builtin_fmaxf(__builtin_fmaxf(s[b][3], s[b][4]), s[b][5]);
      const float m2 = __builtin_fmaxf(__builtin_fmaxf(s[b][6], s[b][7]), s[b][8]);
      const float m3 = __builtin_fmaxf(__builtin_fmaxf(s[b][9], s[b][10]), s[b][11]);
      const float m4 = __builtin_fmaxf(__builtin_fmaxf(s[b][12], s[b][13]), s[b][14]);
      float bm = __builtin_fmaxf(__builtin_fmaxf(__builtin_fmaxf(m0, m1), m2),
                                 __builtin_fmaxf(__builtin_fmaxf(m3, m4), s[b][15]));
      bm = other_half_max(bm);                        // block max relative to base[b]
      const bool up = first || bm > kLazyRescale;
      if (__builtin_amdgcn_ballot_w64(up)) {
        // new base (a bf16 value, so -base is exact in qneg); this block's exponents
        // are moved by the same shift d and earlier blocks rescaled by 2^-d
        const float nbase = up && bm > -INFINITY ? static_cast<float>(static_cast<bf16>(base[b] + bm)) : base[b];
        const float d = nbase - base[b];
        const float alpha = d == 0.f ? 1.0f : __builtin_amdgcn_exp2f(-d);
#pragma unroll
        for (int dd = 0; dd < DT; ++dd) oacc[b][dd] *= alpha;
        lrun[b] *= alpha;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[b][r] -= d;
        base[b] = nbase;
        qneg[b][0] = static_cast<bf16>(hf == 0 ? -nbase : 0.0f);
      }
      float pv[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) pv[r] = __builtin_amdgcn_exp2f(s[b][r]);
      bf16x8 pf[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) pf[r >> 3][r & 7] = static_cast<bf16>(pv[r]);
      // row sum of the bf16-rounded P that P V uses: v_dot2_f32_bf16 against (1, 1), two
      // bf16 values per instruction on two independent chains
      float l0 = 0.f, l1 = 0.f;
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const bf16x2 pair = {pf[r >> 2][2 * (r & 3)], pf[r >> 2][2 * (r & 3) + 1]};
        if (r & 1)
          l1 = __builtin_amdgcn_fdot2_f32_bf16(pair, kOnes2, l1, false);
        else
          l0 = __builtin_amdgcn_fdot2_f32_bf16(pair, kOnes2, l0, false);
      }
      lrun[b] += l0 + l1;
#pragma unroll
      for (int d = 0; d < DT; ++d)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          oacc[b][d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[d][j], pf[j], oacc[b][d], 0, 0, 0);
    }
  };
  using masked = std::integral_constant<bool, true>;
  using unmasked = std::integral_constant<bool, false>;
  if (CAUSAL) {
    for (int kbk = 0; kbk < nkb; ++kbk) key_block(kbk, masked{}, kbk == 0);
  } else {
    const int nfull = p.skv / 32;                    // blocks with 32 valid keys
    for (int kbk = 0; kbk < nfull; ++kbk) key_block(kbk, unmasked{}, kbk == 0);
    if (nfull < nkb) key_block(nfull, masked{}, nfull == 0);
  }

  // ---- O = (O^T / l)^T: lane holds query l%32, dh rows 8 (r/4) + 4 (l/32) + r%4 (+32 d) ----
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const float lt = other_half_sum(lrun[b]);
    const int q = qrow[b] + l32;
    if (q >= p.sq) continue;
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        bf16x4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = from_f32<bf16>(oacc[b][d][4 * g4 + e] * inv);
        *reinterpret_cast<bf16x4*>(ob + static_cast<int64_t>(q) * p.o_ss + d * 32 + g4 * 8 + 4 * hf) = o4;
      }
  }
}

template <int DH, int W>
int32_t launch_res(AttnParams p, int skvp, hipStream_t st) {
  p.q_tiles = static_cast<int>(cdiv(p.sq, W * 64));
  const int64_t blocks = static_cast<int64_t>(p.nb) * p.heads * p.q_tiles;
  if (blocks >= 0x7fffffffll) return set_error(WC_ERR_LIMIT, "wc_attention: too many tiles");
  const size_t lds = res_lds_bytes(DH, skvp);
  auto kernel = p.causal ? attn_res_kernel<DH, W, true> : attn_res_kernel<DH, W, false>;
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess)
      return set_error(static_cast<int32_t>(e), "wc_attention: LDS of %zu bytes refused: %s", lds,
                       hipGetErrorString(e));
  }
  kernel<<<dim3(static_cast<uint32_t>(blocks)), dim3(W * 64), lds, st>>>(p, skvp);
  return check_launch("wc_attention");
}

template <typename T, int DH>
int32_t launch_attn_dh(const AttnParams& p, dim3 grid, hipStream_t st) {
  constexpr bool BF = sizeof(T) == 2;
  constexpr size_t lds = sizeof(T) * 2 * (static_cast<size_t>(kBK) * ((DH < 32 ? 32 : DH) + (BF ? 8 : 4)) +
                                          static_cast<size_t>(DH) * (kBK + (BF ? 8 : 4)));
  auto kernel = attn_kernel<T, DH>;
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess)
      return set_error(static_cast<int32_t>(e), "wc_attention: LDS of %zu bytes refused: %s", lds,
                       hipGetErrorString(e));
  }
  kernel<<<grid, kAttnThreads, lds, st>>>(p);
  return check_launch("wc_attention");
}

template <typename T>
int32_t launch_attn(const AttnParams& p, int dh, hipStream_t st) {
  const int64_t blocks = static_cast<int64_t>(p.nb) * p.heads * p.q_tiles;
  if (blocks >= 0x7fffffffll) return set_error(WC_ERR_LIMIT, "wc_attention: too many tiles");
  const dim3 grid(static_cast<uint32_t>(blocks));
  switch (dh) {
    case 16: return launch_attn_dh<T, 16>(p, grid, st);
    case 32: return launch_attn_dh<T, 32>(p, grid, st);
    case 64: return launch_attn_dh<T, 64>(p, grid, st);
    case 128: return launch_attn_dh<T, 128>(p, grid, st);
    default: return set_error(WC_ERR_LIMIT, "wc_attention: head dim %d unsupported (16, 32, 64, 128)", dh);
  }
}

}  // namespace
}  // namespace wc

using namespace wc;

extern "C" int32_t wc_attention(const wc_attn_args* a, void* stream) {
  clear_error();
  WC_REQUIRE(a != nullptr, WC_ERR_NULL, "wc_attention: null args");
  WC_REQUIRE(a->dtype == WC_F32 || a->dtype == WC_BF16 || a->dtype == WC_F16, WC_ERR_DTYPE,
             "wc_attention: unsupported dtype %s", dtype_name(a->dtype));
  WC_REQUIRE(a->nb >= 0 && a->heads > 0 && a->sq >= 0 && a->skv >= 0 && a->head_dim > 0, WC_ERR_SHAPE,
             "wc_attention: bad sizes");
  if (a->nb == 0 || a->sq == 0) return WC_OK;
  WC_REQUIRE(a->skv > 0, WC_ERR_SHAPE, "wc_attention: no keys");
  WC_REQUIRE(a->q && a->k && a->v && a->o, WC_ERR_NULL, "wc_attention: null pointer");
  const int es = dtype_size(a->dtype);
  const bool al = aligned(a->q, 16) && aligned(a->k, 16) && aligned(a->v, 16) &&
                  (a->q_stride_nb * es) % 16 == 0 && (a->q_stride_s * es) % 16 == 0 &&
                  (a->k_stride_nb * es) % 16 == 0 && (a->k_stride_s * es) % 16 == 0 &&
                  (a->v_stride_nb * es) % 16 == 0 && (a->v_stride_s * es) % 16 == 0;
  WC_REQUIRE(al, WC_ERR_ALIGN, "wc_attention: q/k/v rows must be 16-byte aligned");
  WC_REQUIRE(a->sq < 0x7fffffffll && a->skv < 0x7fffffffll && a->nb < 0x7fffffffll, WC_ERR_LIMIT,
             "wc_attention: sizes too large");
  AttnParams p;
  p.nb = (int)a->nb;
  p.heads = (int)a->heads;
  p.sq = (int)a->sq;
  p.skv = (int)a->skv;
  p.causal = a->causal ? 1 : 0;
  p.q_tiles = static_cast<int>(cdiv(a->sq, kBQ));
  p.scale_log2 = a->scale * 1.4426950408889634f;
  p.q = a->q;
  p.q_sb = a->q_stride_nb;
  p.q_ss = a->q_stride_s;
  p.k = a->k;
  p.k_sb = a->k_stride_nb;
  p.k_ss = a->k_stride_s;
  p.v = a->v;
  p.v_sb = a->v_stride_nb;
  p.v_ss = a->v_stride_s;
  p.o = a->o;
  p.o_sb = a->o_stride_nb;
  p.o_ss = a->o_stride_s;
  p.mask = static_cast<const float*>(a->mask);
  p.m_sb = a->mask_stride_nb;
  p.m_sh = a->mask_stride_head;
  p.m_sq = a->mask_stride_q;
  if (p.mask) {
    WC_REQUIRE(a->mask_stride_nb >= 0 && a->mask_stride_head >= 0 && a->mask_stride_q >= 0, WC_ERR_ARG,
               "wc_attention: negative mask stride");
    WC_REQUIRE(!a->causal, WC_ERR_ARG, "wc_attention: a mask and causal masking are exclusive");
  }
  if (!p.mask && a->dtype == WC_BF16 && (a->head_dim == 32 || a->head_dim == 64)) {
    // resident-KV kernel: K and V of one head in LDS, 8-byte aligned output rows
    const int skvp = static_cast<int>(cdiv(a->skv, 32) * 32);
    const bool o_al = aligned(a->o, 8) && (a->o_stride_nb * es) % 8 == 0 && (a->o_stride_s * es) % 8 == 0;
    if (o_al && res_lds_bytes((int)a->head_dim, skvp) <= 150 * 1024) {
      const bool w8 = a->sq > 256;
      if (a->head_dim == 32)
        return w8 ? launch_res<32, 8>(p, skvp, as_stream(stream)) : launch_res<32, 4>(p, skvp, as_stream(stream));
      return w8 ? launch_res<64, 8>(p, skvp, as_stream(stream)) : launch_res<64, 4>(p, skvp, as_stream(stream));
    }
  }
  if (a->dtype == WC_BF16) return launch_attn<bf16>(p, (int)a->head_dim, as_stream(stream));
  if (a->dtype == WC_F16) return launch_attn<f16>(p, (int)a->head_dim, as_stream(stream));
  return launch_attn<float>(p, (int)a->head_dim, as_stream(stream));
}
