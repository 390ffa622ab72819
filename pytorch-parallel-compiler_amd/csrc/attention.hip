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
  // head dims other than the kernel's own (attn_kernel with GEN): the true head dim, and the
  // first head-dim column of the output chunk this launch computes
  int dh, oc0;
};

constexpr int kAttnThreads = 256;
constexpr int kBQ = 128;   // queries per workgroup (32 per wave)
constexpr int kBK = 64;    // keys per tile

__device__ __forceinline__ float xor_max(float v, int m) { return fmaxf(v, __shfl_xor(v, m, 64)); }
__device__ __forceinline__ float xor_sum(float v, int m) { return v + __shfl_xor(v, m, 64); }

// DH: the head dim of the scores (a multiple of 16, padded to 32 inside); DO: the head-dim
// columns of V and O one launch computes (DH unless GEN).  GEN: the true head dim p.dh may be
// any value up to DH, its rows need no alignment, and this launch computes output columns
// [p.oc0, p.oc0 + DO) of each head: every load and store is element-wise, with the columns
// past p.dh read as zero and not written.
// At least two waves per SIMD (VGPRs + AGPRs within 256) where that compiles without scratch,
// and for the exact 16-bit 128-wide tile, whose ~92 bytes of spills cost less than the second
// wave gains: left to itself the compiler gives that tile 254 + 64 registers, one wave per SIMD
// (2048 tokens, bf16: head dim 64 0.93 -> 0.68 ms, 128 2.87 -> 2.12 ms).  The general 128-wide
// tile and fp32 past 64 would spill without gaining; they keep the compiler's choice.
template <typename T, int DH, bool GEN>
constexpr int attn_min_waves() {
  if constexpr (sizeof(T) == 2) return (DH <= 96 || (DH == 128 && !GEN)) ? 2 : 1;
  else return DH <= 64 ? 2 : 1;
}

template <typename T, int DH, bool GEN = false, int DO = DH, bool VEC = false>
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(attn_min_waves<T, DH, GEN>())))
void attn_kernel(AttnParams p) {
  static_assert(GEN || DO == DH, "only the general form splits the output columns");
  static_assert(GEN || !VEC, "VEC selects the general form's 16-byte loads");
  constexpr bool BF = sizeof(T) == 2;
  constexpr int DHP = DH < 32 ? 32 : DH;       // head dim padded to the 32-wide S^T k-step
  constexpr int KP = DHP + (BF ? 8 : 4);       // K tile pitch (elements)
  constexpr int VP = kBK + (BF ? 8 : 4);       // V^T tile pitch (elements)
  constexpr int DT = DO / 16;                  // 16-row tiles of O^T
  constexpr int NKS = DHP / 32;                // 32-wide head-dim steps of S^T = K Q^T
  extern __shared__ float4 smem4[];
  T* const ks0 = reinterpret_cast<T*>(smem4);   // [2][kBK * KP]  K tiles
  T* const vt0 = ks0 + 2 * kBK * KP;            // [2][DO * VP]   V^T tiles

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int fr = lane & 15, g = lane >> 4;
  // Workgroups are dealt to the 8 XCDs round-robin.  Give XCD x the contiguous range
  // [x * grid/8, (x+1) * grid/8) of (head, query tile) pairs, so a head's query tiles share one
  // L2 (its K/V is fetched once per XCD, not by every XCD) and every XCD gets every tile
  // length under a causal mask; within a head the last (longest causal) tiles start first.
  int lin = blockIdx.x;
  if ((gridDim.x & 7) == 0) lin = (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
  const int bh = lin / p.q_tiles;
  const int qt = p.q_tiles - 1 - (lin - bh * p.q_tiles);
  const int nb = bh / p.heads, h = bh - (bh / p.heads) * p.heads;
  const int hd = GEN ? p.dh : DH;               // head stride within a row
  const int oc0 = GEN ? p.oc0 : 0;              // first V / O column of this launch
  const T* qb = static_cast<const T*>(p.q) + nb * p.q_sb + h * hd;
  const T* kb = static_cast<const T*>(p.k) + nb * p.k_sb + h * hd;
  const T* vb = static_cast<const T*>(p.v) + nb * p.v_sb + h * hd + oc0;
  T* ob = static_cast<T*>(p.o) + nb * p.o_sb + h * hd + oc0;
  const int q0 = qt * kBQ + wave * 32;           // first query of this wave
  const T tzero = from_f32<T>(0.f);

  // ---- Q^T fragments (B operand of S^T = K Q^T), kept in registers ----
  // lane supplies Q[q = q0 + nt*16 + fr][d = s*32 + g*8 .. +8] (fp32: two 16-byte halves)
  uint4 qf[2][NKS][2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int q = q0 + nt * 16 + fr;
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      const T* src = qb + q * p.q_ss + s * 32 + g * 8;
      if constexpr (GEN && VEC) {
        // the head dim is a whole number of 16-byte pieces: each lies inside it or past it
        const int c = s * 32 + g * 8;
        qf[nt][s][0] = (q < p.sq && c < hd) ? *reinterpret_cast<const uint4*>(src) : make_uint4(0, 0, 0, 0);
        qf[nt][s][1] = (!BF && q < p.sq && c + 4 < hd) ? *reinterpret_cast<const uint4*>(src + (BF ? 0 : 4))
                                                        : make_uint4(0, 0, 0, 0);
      } else if constexpr (GEN) {
        T t8[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) t8[j] = (q < p.sq && s * 32 + g * 8 + j < hd) ? src[j] : tzero;
        __builtin_memcpy(&qf[nt][s][0], t8, 16);
        if (BF) qf[nt][s][1] = make_uint4(0, 0, 0, 0);
        else __builtin_memcpy(&qf[nt][s][1], reinterpret_cast<const char*>(t8) + 16, 16);
      } else {
        const bool ok = q < p.sq && s * 32 + g * 8 < DH;   // head-dim padding reads as zero
        qf[nt][s][0] = ok ? *reinterpret_cast<const uint4*>(src) : make_uint4(0, 0, 0, 0);
        qf[nt][s][1] = (!BF && ok) ? *reinterpret_cast<const uint4*>(src + (BF ? 0 : 4)) : make_uint4(0, 0, 0, 0);
      }
    }
  }

  // ---- staging of one K / V tile: each thread moves 16-byte row pieces of each ----
  constexpr int VE = 16 / sizeof(T);
  constexpr int KPIECES = kBK * DH / VE;         // 16-byte pieces per K tile
  constexpr int VPIECES = kBK * DO / VE;         // and per V tile
  constexpr int KPPT = (KPIECES + kAttnThreads - 1) / kAttnThreads;
  constexpr int VPPT = (VPIECES + kAttnThreads - 1) / kAttnThreads;
  uint4 kreg[KPPT], vreg[VPPT];
  // a piece of `cols` valid columns from `src` (element-wise; the rest zero).  VEC: cols is
  // either <= 0 or at least a whole piece, and src is 16-byte aligned
  auto piece = [&](const T* src, int cols) {
    if constexpr (VEC) return cols > 0 ? *reinterpret_cast<const uint4*>(src) : make_uint4(0, 0, 0, 0);
    T t[VE];
#pragma unroll
    for (int j = 0; j < VE; ++j) t[j] = j < cols ? src[j] : tzero;
    uint4 u;
    __builtin_memcpy(&u, t, 16);
    return u;
  };
  auto fetch = [&](int k0) {
    if constexpr (!GEN) {
      // K and V pieces share their (key, column) here (DO == DH)
#pragma unroll
      for (int u = 0; u < KPPT; ++u) {
        const int e = tid + u * kAttnThreads;
        const int key = e / (DH / VE), c = (e - key * (DH / VE)) * VE;
        const bool ok = e < KPIECES && k0 + key < p.skv;
        kreg[u] = ok ? *reinterpret_cast<const uint4*>(kb + (k0 + key) * p.k_ss + c) : make_uint4(0, 0, 0, 0);
        vreg[u] = ok ? *reinterpret_cast<const uint4*>(vb + (k0 + key) * p.v_ss + c) : make_uint4(0, 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int u = 0; u < KPPT; ++u) {
        const int e = tid + u * kAttnThreads;
        const int key = e / (DH / VE), c = (e - key * (DH / VE)) * VE;
        const bool ok = e < KPIECES && k0 + key < p.skv;
        kreg[u] = ok ? piece(kb + (k0 + key) * p.k_ss + c, hd - c) : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < VPPT; ++u) {
        const int e = tid + u * kAttnThreads;
        const int key = e / (DO / VE), c = (e - key * (DO / VE)) * VE;
        const bool ok = e < VPIECES && k0 + key < p.skv;
        vreg[u] = ok ? piece(vb + (k0 + key) * p.v_ss + c, hd - oc0 - c) : make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto stash = [&](int buf) {
    if constexpr (!GEN) {
#pragma unroll
      for (int u = 0; u < KPPT; ++u) {
        const int e = tid + u * kAttnThreads;
        if (e >= KPIECES) continue;
        const int key = e / (DH / VE), c = (e - key * (DH / VE)) * VE;
        *reinterpret_cast<uint4*>(&ks0[buf * kBK * KP + key * KP + c]) = kreg[u];
        const T* vv = reinterpret_cast<const T*>(&vreg[u]);
#pragma unroll
        for (int q = 0; q < VE; ++q) vt0[buf * DH * VP + (c + q) * VP + key] = vv[q];
      }
    } else {
#pragma unroll
      for (int u = 0; u < KPPT; ++u) {
        const int e = tid + u * kAttnThreads;
        if (e >= KPIECES) continue;
        const int key = e / (DH / VE), c = (e - key * (DH / VE)) * VE;
        *reinterpret_cast<uint4*>(&ks0[buf * kBK * KP + key * KP + c]) = kreg[u];
      }
#pragma unroll
      for (int u = 0; u < VPPT; ++u) {
        const int e = tid + u * kAttnThreads;
        if (e >= VPIECES) continue;
        const int key = e / (DO / VE), c = (e - key * (DO / VE)) * VE;
        const T* vv = reinterpret_cast<const T*>(&vreg[u]);
#pragma unroll
        for (int q = 0; q < VE; ++q) vt0[buf * DO * VP + (c + q) * VP + key] = vv[q];
      }
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
    const T* vt_s = vt0 + buf * DO * VP;

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
      for (int e = 0; e < 4; ++e)
        if (!GEN || oc0 + dt * 16 + g * 4 + e < hd) dst[e] = from_f32<T>(acc_o[dt][nt][e] * inv);
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
//                    halves through the lane crossbar; the running max
//                    only moves when a block exceeds it by 2^8 (P <= 2^8 keeps
//                    fp32 sums exact enough), so most blocks skip the rescale
//   O^T += V^T P^T   P^T is the S^T register block itself: k-step j takes
//                    registers 8j..8j+7, i.e. keys 16j + 8 (s/4) + 4 (l/32) + s%4,
//                    and V^T is read from LDS in that key order (two 8-byte reads)
// Scores are scaled by log2(e)/sqrt(Dh) inside the exp2 argument (one FMA).
// ---------------------------------------------------------------------------
constexpr float kLazyRescale = 8.0f;
constexpr bf16x2 kOnes2 = {bf16(1.0f), bf16(1.0f)};

// (v of this lane, v of lane l ^ 32) through the lane crossbar (ds_bpermute_b32).
// The half-wave swap instruction (v_permlane32_swap) is not used: its 16-lane sibling
// delivered a stale first word now and then in the conv epilogue, with the compiler's
// wait states around it, and a stale softmax max or row sum would corrupt whole rows.
__device__ __forceinline__ void half_swap(float v, float& mine, float& other) {
  mine = v;
  other = __shfl_xor(v, 32, 64);
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

// The key loop of attn_res_kernel as functions, for attn_qkv_kernel.  attn_res_kernel keeps its
// own inline copy: its causal variant compiled through these functions takes 136 VGPRs
// instead of 121, which costs a wave per SIMD.
//
// One wave's two 32-query blocks in the resident-KV key loop: the Q^T fragments (B operand of
// S^T = K Q^T, pre-scaled by scale * log2(e)), the row of -base that the extra k-step adds
// (qneg: B operand, k = 0 of the lanes < 32), the O^T accumulators, and per query row the
// running base (a bf16 value, 0 until the first block sets it) and the running sum.
template <int NKS, int DT>
struct ResRows {
  bf16x8 qf[2][NKS];
  bf16x8 qneg[2];
  f32x16 oacc[2][DT];
  float base[2], lrun[2];
};

template <int NKS, int DT>
__device__ __forceinline__ void res_rows_init(ResRows<NKS, DT>& r) {
#pragma unroll
  for (int b = 0; b < 2; ++b) {
#pragma unroll
    for (int e = 0; e < 8; ++e) r.qneg[b][e] = static_cast<bf16>(0.0f);
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int e = 0; e < 16; ++e) r.oacc[b][d][e] = 0.f;
    r.base[b] = 0.f;
    r.lrun[b] = 0.f;
  }
}

// K extended by a column of ones: A operand of the extra k-step, k = 0 of the lanes < 32
__device__ __forceinline__ bf16x8 res_kone(int hf) {
  bf16x8 kone;
#pragma unroll
  for (int e = 0; e < 8; ++e) kone[e] = static_cast<bf16>(e == 0 && hf == 0 ? 1.0f : 0.0f);
  return kone;
}

// One 32-key block starting at key0, for both query blocks (first queries qrow[0], qrow[1]).  kf: A fragments of S^T = K Q^T
// (lane: key key0 + l%32, k-step k).  vf: A fragments of O^T += V^T P^T (lane: head dim
// 32 d + l%32; k-step j takes the keys of S^T registers 8 j .. 8 j + 7, i.e. keys
// 16 j + 8 (e / 4) + 4 (l / 32) + e % 4 of the block).  Both query blocks' scores come
// first (their MFMA latency hides behind the first block's softmax), then per query block
// the softmax and P V.
template <int NKS, int DT, bool CAUSAL, bool MASK>
__device__ __forceinline__ void res_key_block(ResRows<NKS, DT>& r, const int (&qrow)[2], const bf16x8 (&kf)[NKS],
                                              const bf16x8 (&vf)[DT][2], const bf16x8& kone, int key0,
                                              bool first, int skv, int hf, int l32) {
  f32x16 s[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    if (CAUSAL && key0 > qrow[b] + 31) continue;
#pragma unroll
    for (int e = 0; e < 16; ++e) s[b][e] = 0.f;
#pragma unroll
    for (int k = 0; k < NKS; ++k) s[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[k], r.qf[b][k], s[b], 0, 0, 0);
    s[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kone, r.qneg[b], s[b], 0, 0, 0);
  }
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    if (CAUSAL && key0 > qrow[b] + 31) continue;
    if constexpr (MASK) {
      const int q = qrow[b] + l32;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = key0 + (i >> 2) * 8 + 4 * hf + (i & 3);
        if (key >= skv || (CAUSAL && key > q)) s[b][i] = -INFINITY;
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
    bm = other_half_max(bm);                          // block max relative to base[b]
    const bool up = first || bm > kLazyRescale;
    if (__builtin_amdgcn_ballot_w64(up)) {
      // new base (a bf16 value, so -base is exact in qneg); this block's exponents
      // are moved by the same shift d and earlier blocks rescaled by 2^-d
      const float nbase = up && bm > -INFINITY ? static_cast<float>(static_cast<bf16>(r.base[b] + bm)) : r.base[b];
      const float d = nbase - r.base[b];
      const float alpha = d == 0.f ? 1.0f : __builtin_amdgcn_exp2f(-d);
#pragma unroll
      for (int dd = 0; dd < DT; ++dd) r.oacc[b][dd] *= alpha;
      r.lrun[b] *= alpha;
#pragma unroll
      for (int i = 0; i < 16; ++i) s[b][i] -= d;
      r.base[b] = nbase;
      r.qneg[b][0] = static_cast<bf16>(hf == 0 ? -nbase : 0.0f);
    }
    float pv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) pv[i] = __builtin_amdgcn_exp2f(s[b][i]);
    bf16x8 pf[2];
#pragma unroll
    for (int i = 0; i < 16; ++i) pf[i >> 3][i & 7] = static_cast<bf16>(pv[i]);
    // row sum of the bf16-rounded P that P V uses: v_dot2_f32_bf16 against (1, 1), two
    // bf16 values per instruction on two independent chains
    float l0 = 0.f, l1 = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bf16x2 pair = {pf[i >> 2][2 * (i & 3)], pf[i >> 2][2 * (i & 3) + 1]};
      if (i & 1)
        l1 = __builtin_amdgcn_fdot2_f32_bf16(pair, kOnes2, l1, false);
      else
        l0 = __builtin_amdgcn_fdot2_f32_bf16(pair, kOnes2, l0, false);
    }
    r.lrun[b] += l0 + l1;
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        r.oacc[b][d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[d][j], pf[j], r.oacc[b][d], 0, 0, 0);
  }
}

// O = (O^T / l)^T: lane holds query qrow[b] + l%32, head dims 8 (i/4) + 4 (l/32) + i%4 (+32 d)
// of register i; ob points at head dim 0 of query 0
template <int NKS, int DT>
__device__ __forceinline__ void res_store_o(const ResRows<NKS, DT>& r, const int (&qrow)[2], bf16* ob, int64_t o_ss,
                                            int sq, int hf, int l32) {
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const float lt = other_half_sum(r.lrun[b]);
    const int q = qrow[b] + l32;
    if (q >= sq) continue;
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        bf16x4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = from_f32<bf16>(r.oacc[b][d][4 * g4 + e] * inv);
        *reinterpret_cast<bf16x4*>(ob + static_cast<int64_t>(q) * o_ss + d * 32 + g4 * 8 + 4 * hf) = o4;
      }
  }
}

template <int DH, int W, bool CAUSAL>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(W == 4 ? 2 : 1))) void attn_res_kernel(AttnParams p, int skvp) {
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
    // only the blocks on a query block's diagonal, or past the last key, need the mask
    for (int kbk = 0; kbk < nkb; ++kbk) {
      const int key0 = kbk * 32;
      if ((key0 + 31 > qrow[0] && key0 <= qrow[0] + 31) || key0 + 31 > qrow[1] || key0 + 32 > p.skv)
        key_block(kbk, masked{}, kbk == 0);
      else
        key_block(kbk, unmasked{}, kbk == 0);
    }
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

// ---------------------------------------------------------------------------
// Self-attention with the Q, K and V projections inside (bf16, head dim 32).
// One workgroup per (model*batch, head), holding every token of the row (S <= W*64):
//   phase 1  the head's 96 projection rows (its Q, K and V rows of the weights, D wide)
//            and their biases (fp32, zero when absent) are staged in LDS;
//   phase 2  wave w projects its two 32-token blocks w and 2W-1-w (its query blocks) with
//            v_mfma_f32_32x32x16_bf16, reading x straight from memory (no other wave needs
//            those rows): Q^T = Wq x^T and K^T = Wk x^T (lane: token l%32, head dims
//            8 (i/4) + 4 (l/32) + i%4 in register i) and V = x Wv^T (lane: head dim l%32,
//            tokens 8 (i/4) + 4 (l/32) + i%4).  Registers 8k..8k+7 of Q^T are then the B
//            fragments of k-step k of S^T = K Q^T for the head-dim order
//            16 k + 8 (e/4) + 4 (l/32) + e%4, which the K^T registers share, and registers
//            8j..8j+7 of V are the A fragments of k-step j of O^T += V^T P^T for their key
//            block, so neither needs a lane exchange.  The accumulators start at the bias;
//   phase 3  K and V (rounded to bf16) go to LDS over the weights in fragment
//            order, [32-key block][k-step][lane half][lane%32][8], read back with one
//            conflict-free 16-byte load per fragment;
// then the resident key loop (res_key_block) over the key blocks.
// ---------------------------------------------------------------------------
struct QkvParams {
  int nb, heads, b, s, d;                            // nb = models * b rows; d = model dim
  float scale_log2;
  const bf16* x;
  int64_t x_sn, x_sb, x_ss;
  const bf16* wq;                                    // [models][d][d]
  int64_t wq_sn;
  const bf16* wkv;                                   // [models][2d][d]: K rows, then V rows
  int64_t wkv_sn;
  const bf16* bq;                                    // [models][d] or null
  int64_t bq_sn;
  const bf16* bkv;                                   // [models][2d] or null
  int64_t bkv_sn;
  bf16* o;
  int64_t o_sb, o_ss;
  // workgroups [stagger_lo, stagger_hi) (the second workgroup of each CU in the first round of
  // dispatch) start after a pause; 0, 0 = none
  int stagger_lo, stagger_hi;
};

constexpr int kQkvRows = 96;                         // Q, K and V rows of one head (head dim 32)
constexpr int kQkvBlockElems = 1024;                 // K (or V) fragments of one 32-key block

inline size_t qkv_lds_bytes(int d, int w) {
  // phases 1-2: the weight rows, then their 96 biases in fp32
  const size_t wts = static_cast<size_t>(kQkvRows) * (d + 8) * sizeof(bf16) + kQkvRows * sizeof(float);
  const size_t kv = static_cast<size_t>(2 * w) * 2 * kQkvBlockElems * sizeof(bf16);
  return wts > kv ? wts : kv;
}

template <int W, bool CAUSAL>
__global__ __launch_bounds__(W * 64, 4) void attn_qkv_kernel(QkvParams p) {   // 4 waves per SIMD
  constexpr int NKS = 2, DT = 1;                     // head dim 32: two 16-dim k-steps, one O^T tile
  extern __shared__ float4 smem4[];
  bf16* const wsm = reinterpret_cast<bf16*>(smem4);  // phases 1-2: [96][d + 8], then float [96] biases
  bf16* const ksm = wsm;                             // phase 3 on: [2W][NKS][2][32][8]
  bf16* const vsm = wsm + 2 * W * kQkvBlockElems;    //             [2W][2][2][32][8]
  const int wp = p.d + 8;
  float* const bsm = reinterpret_cast<float*>(wsm + kQkvRows * wp);

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, hf = lane >> 5;
  // XCD x takes the contiguous range [x G / 8, (x + 1) G / 8) of (row, head) ids: the heads of
  // one row read its x through one L2, and the rows of one model its weights
  const int G = gridDim.x;
  const int bid = (G & 7) == 0 ? (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  const int nb = bid / p.heads, h = bid - nb * p.heads;
  const int mdl = nb / p.b, bb = nb - mdl * p.b;

  // The two workgroups that share a CU would otherwise run their projections (MFMA and memory)
  // together and then their key loops (VALU) together; starting the second one ~16K cycles
  // later lets one's projection run beside the other's key loop (c. 5% on 16 x 8 x 512 x 256).
  if (static_cast<int>(blockIdx.x) >= p.stagger_lo && static_cast<int>(blockIdx.x) < p.stagger_hi) {
    __builtin_amdgcn_s_sleep(127);
    __builtin_amdgcn_s_sleep(127);
  }

  // ---- phase 1: rows 0-31 = Wq, 32-63 = Wk, 64-95 = Wv rows of head h ----
  {
    const bf16* wq = p.wq + mdl * p.wq_sn + static_cast<int64_t>(h) * 32 * p.d;
    const bf16* wk = p.wkv + mdl * p.wkv_sn + static_cast<int64_t>(h) * 32 * p.d;
    const bf16* wv = wk + static_cast<int64_t>(p.d) * p.d;
    if (tid < kQkvRows) {                            // biases; absent ones are zero
      const bf16* bsrc = tid < 32 ? (p.bq ? p.bq + mdl * p.bq_sn + h * 32 + tid : nullptr)
                                  : (p.bkv ? p.bkv + mdl * p.bkv_sn + (tid < 64 ? 0 : p.d) + h * 32 + (tid & 31)
                                           : nullptr);
      bsm[tid] = bsrc ? static_cast<float>(*bsrc) : 0.f;
    }
    const int cpr = p.d / 8;                         // 16-byte chunks per row
    const int total = kQkvRows * cpr;
    constexpr int U = 4;                             // chunks per thread in flight
    for (int e0 = tid; e0 < total; e0 += U * W * 64) {
      uint4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int e = e0 + u * W * 64;
        const int row = e / cpr, c = (e - row * cpr) * 8;
        const bf16* src = row < 32 ? wq + row * p.d : row < 64 ? wk + (row - 32) * p.d : wv + (row - 64) * p.d;
        v[u] = e < total ? *reinterpret_cast<const uint4*>(src + c) : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int e = e0 + u * W * 64;
        if (e >= total) continue;
        const int row = e / cpr, c = (e - row * cpr) * 8;
        *reinterpret_cast<uint4*>(wsm + row * wp + c) = v[u];
      }
    }
  }
  __syncthreads();

  // ---- phase 2: Q, K, V of the wave's token blocks ----
  const int qrow[2] = {wave * 32, (2 * W - 1 - wave) * 32};
  ResRows<NKS, DT> r;
  bf16x8 kreg[2][NKS], vreg[2][2];
  const float c = p.scale_log2;
  const bf16* xb = p.x + mdl * p.x_sn + bb * p.x_sb;
  const int ksteps = p.d / 16;                       // even: d is a multiple of 32
  // one pass over the k-steps of block b: Q^T if QP, K^T and V if KVP (both, for both blocks)
  auto project = [&](int b, auto qp_tag, auto kvp_tag) {
    constexpr bool QP = decltype(qp_tag)::value, KVP = decltype(kvp_tag)::value;
    // the accumulators start at the bias of their head dims (an fp32 add before the bf16
    // rounding, as in the projection GEMM's epilogue)
    f32x16 aq, ak, av;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4 tq = QP ? *reinterpret_cast<const f32x4*>(bsm + 8 * i + 4 * hf) : f32x4{};
      const f32x4 tk = KVP ? *reinterpret_cast<const f32x4*>(bsm + 32 + 8 * i + 4 * hf) : f32x4{};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        aq[4 * i + e] = tq[e];
        ak[4 * i + e] = tk[e];
      }
    }
    const float bv = KVP ? bsm[64 + l32] : 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) av[e] = bv;
    if (qrow[b] < p.s) {                             // blocks past the last token stay unused
      int tok = qrow[b] + l32;
      tok = tok < p.s ? tok : p.s - 1;
      const bf16* xr = xb + static_cast<int64_t>(tok) * p.x_ss + 8 * hf;
      const bf16* wr = wsm + l32 * wp + 8 * hf;
      bf16x8 xa[2], xn[2];
      xa[0] = *reinterpret_cast<const bf16x8*>(xr);
      xa[1] = *reinterpret_cast<const bf16x8*>(xr + 16);
      for (int s = 0; s < ksteps; s += 2) {
        xn[0] = xa[0];
        xn[1] = xa[1];
        if (s + 2 < ksteps) {                        // next pair of k-steps in flight
          xn[0] = *reinterpret_cast<const bf16x8*>(xr + 16 * (s + 2));
          xn[1] = *reinterpret_cast<const bf16x8*>(xr + 16 * (s + 3));
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const bf16* w = wr + 16 * (s + u);
          if constexpr (QP) {
            const bf16x8 fq = *reinterpret_cast<const bf16x8*>(w);
            aq = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fq, xa[u], aq, 0, 0, 0);
          }
          if constexpr (KVP) {
            const bf16x8 fk = *reinterpret_cast<const bf16x8*>(w + 32 * wp);
            const bf16x8 fv = *reinterpret_cast<const bf16x8*>(w + 64 * wp);
            ak = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fk, xa[u], ak, 0, 0, 0);
            av = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[u], fv, av, 0, 0, 0);
          }
        }
        xa[0] = xn[0];
        xa[1] = xn[1];
      }
    }
    // Q is pre-scaled by scale * log2(e) after its bf16 rounding and rounded again, as
    // attn_res_kernel does with the Q it reads
#pragma unroll
    for (int k = 0; k < NKS; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int i = 8 * k + e;
        if constexpr (QP) r.qf[b][k][e] = static_cast<bf16>(static_cast<float>(static_cast<bf16>(aq[i])) * c);
        if constexpr (KVP) {
          kreg[b][k][e] = static_cast<bf16>(ak[i]);
          vreg[b][k][e] = static_cast<bf16>(av[i]);
        }
      }
  };
  using yes = std::integral_constant<bool, true>;
  project(0, yes{}, yes{});
  project(1, yes{}, yes{});
  __syncthreads();                                   // every wave is done with the weights

  // ---- phase 3: K and V of the wave's blocks into LDS, fragment order ----
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int kb = qrow[b] / 32;
#pragma unroll
    for (int k = 0; k < NKS; ++k)
      *reinterpret_cast<bf16x8*>(ksm + (((kb * NKS + k) * 2 + hf) * 32 + l32) * 8) = kreg[b][k];
#pragma unroll
    for (int j = 0; j < 2; ++j)
      *reinterpret_cast<bf16x8*>(vsm + (((kb * 2 + j) * 2 + hf) * 32 + l32) * 8) = vreg[b][j];
  }
  const bf16x8 kone = res_kone(hf);
  res_rows_init(r);
  __syncthreads();

  const int nkv = (p.s + 31) / 32;                   // key blocks
  int nkb = nkv;
  if (CAUSAL) {
    const int qmax = qrow[1] + 31;                   // qrow[1] >= qrow[0]
    const int last = (qmax < p.s ? qmax : p.s - 1) / 32 + 1;
    nkb = last < nkb ? last : nkb;
  }
  auto key_block = [&](int kbk, auto mask_tag, bool first) {
    constexpr bool MASK = decltype(mask_tag)::value;
    bf16x8 kf[NKS];
#pragma unroll
    for (int k = 0; k < NKS; ++k)
      kf[k] = *reinterpret_cast<const bf16x8*>(ksm + (((kbk * NKS + k) * 2 + hf) * 32 + l32) * 8);
    bf16x8 vf[DT][2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
      vf[0][j] = *reinterpret_cast<const bf16x8*>(vsm + (((kbk * 2 + j) * 2 + hf) * 32 + l32) * 8);
    res_key_block<NKS, DT, CAUSAL, MASK>(r, qrow, kf, vf, kone, kbk * 32, first, p.s, hf, l32);
  };
  using masked = std::integral_constant<bool, true>;
  using unmasked = std::integral_constant<bool, false>;
  if (CAUSAL) {
    // only the blocks on a query block's diagonal, or past the last key, need the mask
    for (int kbk = 0; kbk < nkb; ++kbk) {
      const int key0 = kbk * 32;
      if ((key0 + 31 > qrow[0] && key0 <= qrow[0] + 31) || key0 + 31 > qrow[1] || key0 + 32 > p.s)
        key_block(kbk, masked{}, kbk == 0);
      else
        key_block(kbk, unmasked{}, kbk == 0);
    }
  } else {
    const int nfull = p.s / 32;                      // blocks with 32 valid keys
    for (int kbk = 0; kbk < nfull; ++kbk) key_block(kbk, unmasked{}, kbk == 0);
    if (nfull < nkb) key_block(nfull, masked{}, nfull == 0);
  }
  res_store_o(r, qrow, p.o + nb * p.o_sb + h * 32, p.o_ss, p.s, hf, l32);
}

template <int W>
int32_t launch_qkv(QkvParams p, bool causal, hipStream_t st) {
  const int64_t blocks = static_cast<int64_t>(p.nb) * p.heads;
  if (blocks >= 0x7fffffffll) return set_error(WC_ERR_LIMIT, "wc_self_attention: too many (row, head) pairs");
  const size_t lds = qkv_lds_bytes(p.d, W);
  // two eight-wave workgroups per CU (LDS and four waves per SIMD allow no more): stagger the
  // second ones, dispatched after one workgroup has gone to every CU
  const int cus = device_cu_count();
  p.stagger_lo = p.stagger_hi = 0;
  if (W == 8 && cus > 0 && lds * 2 <= 160 * 1024 && blocks > cus) {
    p.stagger_lo = cus;
    p.stagger_hi = 2 * cus;
  }
  auto kernel = causal ? attn_qkv_kernel<W, true> : attn_qkv_kernel<W, false>;
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess)
      return set_error(static_cast<int32_t>(e), "wc_self_attention: LDS of %zu bytes refused: %s", lds,
                       hipGetErrorString(e));
  }
  kernel<<<dim3(static_cast<uint32_t>(blocks)), dim3(W * 64), lds, st>>>(p);
  return check_launch("wc_self_attention");
}

template <typename T, int DH, bool GEN = false, int DO = DH, bool VEC = false>
int32_t launch_attn_dh(const AttnParams& p, dim3 grid, hipStream_t st) {
  constexpr bool BF = sizeof(T) == 2;
  constexpr size_t lds = sizeof(T) * 2 * (static_cast<size_t>(kBK) * ((DH < 32 ? 32 : DH) + (BF ? 8 : 4)) +
                                          static_cast<size_t>(DO) * (kBK + (BF ? 8 : 4)));
  static_assert(lds <= 160 * 1024, "LDS");
  auto kernel = attn_kernel<T, DH, GEN, DO, VEC>;
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

// The general form: the head dim padded to the next of 16, 32, 64, 96, 128 (256 for 16-bit
// types, computed in output chunks of 128 columns, one launch per chunk, each recomputing the
// scores).  VEC: 16-byte loads (the head dim a whole number of 16-byte pieces, rows aligned).
template <typename T, bool VEC>
int32_t launch_gen(AttnParams p, int dh, dim3 grid, hipStream_t st) {
  if (dh <= 16) return launch_attn_dh<T, 16, true, 16, VEC>(p, grid, st);
  if (dh <= 32) return launch_attn_dh<T, 32, true, 32, VEC>(p, grid, st);
  if (dh <= 64) return launch_attn_dh<T, 64, true, 64, VEC>(p, grid, st);
  if (dh <= 96) return launch_attn_dh<T, 96, true, 96, VEC>(p, grid, st);
  if (dh <= 128) return launch_attn_dh<T, 128, true, 128, VEC>(p, grid, st);
  if constexpr (sizeof(T) == 2) {
    for (int oc0 = 0; oc0 < dh; oc0 += 128) {
      p.oc0 = oc0;
      const int32_t rc = launch_attn_dh<T, 256, true, 128, VEC>(p, grid, st);
      if (rc != WC_OK) return rc;
    }
  }
  return WC_OK;
}

// Head dims 16, 32, 64 and 128 with 16-byte aligned rows take the vector form; any other head
// dim (up to 256 for 16-bit types, 128 for fp32, whose 256-wide K tiles would not fit in LDS),
// or unaligned rows, the general form above.
template <typename T>
int32_t launch_attn(AttnParams p, int dh, bool aligned_rows, hipStream_t st) {
  const int64_t blocks = static_cast<int64_t>(p.nb) * p.heads * p.q_tiles;
  if (blocks >= 0x7fffffffll) return set_error(WC_ERR_LIMIT, "wc_attention: too many tiles");
  const dim3 grid(static_cast<uint32_t>(blocks));
  if (aligned_rows) {
    switch (dh) {
      case 16: return launch_attn_dh<T, 16>(p, grid, st);
      case 32: return launch_attn_dh<T, 32>(p, grid, st);
      case 64: return launch_attn_dh<T, 64>(p, grid, st);
      case 128: return launch_attn_dh<T, 128>(p, grid, st);
      default: break;
    }
  }
  constexpr int kMaxDh = sizeof(T) == 2 ? 256 : 128;
  if (dh > kMaxDh)
    return set_error(WC_ERR_LIMIT, "wc_attention: head dim %d above %d unsupported for %s", dh, kMaxDh,
                     sizeof(T) == 2 ? "16-bit types" : "fp32");
  p.dh = dh;
  p.oc0 = 0;
  // whole 16-byte pieces per head (and 16-byte aligned rows): vector loads
  if (aligned_rows && (dh * static_cast<int>(sizeof(T))) % 16 == 0) return launch_gen<T, true>(p, dh, grid, st);
  return launch_gen<T, false>(p, dh, grid, st);
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
                  ubytes(a->q_stride_nb, es) % 16 == 0 && ubytes(a->q_stride_s, es) % 16 == 0 &&
                  ubytes(a->k_stride_nb, es) % 16 == 0 && ubytes(a->k_stride_s, es) % 16 == 0 &&
                  ubytes(a->v_stride_nb, es) % 16 == 0 && ubytes(a->v_stride_s, es) % 16 == 0;
  WC_REQUIRE(aligned(a->q, es) && aligned(a->k, es) && aligned(a->v, es) && aligned(a->o, es), WC_ERR_ALIGN,
             "wc_attention: q/k/v/o must be aligned to their element size");
  // head offsets within a row (head * head_dim) are 32-bit in the kernels
  WC_REQUIRE(a->head_dim < 0x7fffffffll && a->heads < 0x7fffffffll && a->heads * a->head_dim < 0x7fffffffll,
             WC_ERR_LIMIT, "wc_attention: heads x head dim too large");
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
  p.dh = (int)a->head_dim;
  p.oc0 = 0;
  if (al && !p.mask && a->dtype == WC_BF16 && (a->head_dim == 32 || a->head_dim == 64)) {
    // resident-KV kernel: K and V of one head in LDS, 8-byte aligned output rows
    const int skvp = static_cast<int>(cdiv(a->skv, 32) * 32);
    const bool o_al = aligned(a->o, 8) && ubytes(a->o_stride_nb, es) % 8 == 0 && ubytes(a->o_stride_s, es) % 8 == 0;
    if (o_al && res_lds_bytes((int)a->head_dim, skvp) <= 150 * 1024) {
      const bool w8 = a->sq > 256;
      if (a->head_dim == 32)
        return w8 ? launch_res<32, 8>(p, skvp, as_stream(stream)) : launch_res<32, 4>(p, skvp, as_stream(stream));
      return w8 ? launch_res<64, 8>(p, skvp, as_stream(stream)) : launch_res<64, 4>(p, skvp, as_stream(stream));
    }
  }
  if (a->dtype == WC_BF16) return launch_attn<bf16>(p, (int)a->head_dim, al, as_stream(stream));
  if (a->dtype == WC_F16) return launch_attn<f16>(p, (int)a->head_dim, al, as_stream(stream));
  return launch_attn<float>(p, (int)a->head_dim, al, as_stream(stream));
}

extern "C" int32_t wc_self_attention(const wc_self_attn_args* a, void* stream) {
  clear_error();
  WC_REQUIRE(a != nullptr, WC_ERR_NULL, "wc_self_attention: null args");
  WC_REQUIRE(a->dtype == WC_BF16, WC_ERR_LIMIT, "wc_self_attention: dtype %s (the fused kernel is bf16 only)",
             dtype_name(a->dtype));
  WC_REQUIRE(a->n >= 0 && a->b >= 0 && a->s >= 0 && a->d_model > 0 && a->heads > 0, WC_ERR_SHAPE,
             "wc_self_attention: bad sizes");
  WC_REQUIRE(a->d_model % a->heads == 0 && a->d_model / a->heads == 32, WC_ERR_LIMIT,
             "wc_self_attention: head dim %lld (the fused kernel takes 32)",
             static_cast<long long>(a->d_model % a->heads == 0 ? a->d_model / a->heads : 0));
  WC_REQUIRE(a->s <= 512 && a->d_model <= 768, WC_ERR_LIMIT,
             "wc_self_attention: s = %lld, d_model = %lld (the fused kernel takes s <= 512, d_model <= 768)",
             static_cast<long long>(a->s), static_cast<long long>(a->d_model));
  if (a->n == 0 || a->b == 0 || a->s == 0) return WC_OK;
  WC_REQUIRE(a->x && a->q_weight && a->kv_weight && a->o, WC_ERR_NULL, "wc_self_attention: null pointer");
  WC_REQUIRE(mul_sat({a->n, a->b}) < 0x7fffffffll && a->x_stride_n >= 0 && a->x_stride_b >= 0 && a->x_stride_s >= 0 &&
                 a->o_stride_nb >= 0 && a->o_stride_s >= 0 && a->q_weight_stride_n >= 0 &&
                 a->kv_weight_stride_n >= 0 && a->q_bias_stride_n >= 0 && a->kv_bias_stride_n >= 0,
             WC_ERR_ARG, "wc_self_attention: negative stride or too many rows");
  const bool al = aligned(a->x, 16) && aligned(a->q_weight, 16) && aligned(a->kv_weight, 16) &&
                  (a->x_stride_n * 2) % 16 == 0 && (a->x_stride_b * 2) % 16 == 0 && (a->x_stride_s * 2) % 16 == 0 &&
                  (a->q_weight_stride_n * 2) % 16 == 0 && (a->kv_weight_stride_n * 2) % 16 == 0 &&
                  (!a->q_bias || (aligned(a->q_bias, 8) && (a->q_bias_stride_n * 2) % 8 == 0)) &&
                  (!a->kv_bias || (aligned(a->kv_bias, 8) && (a->kv_bias_stride_n * 2) % 8 == 0)) &&
                  aligned(a->o, 8) && (a->o_stride_nb * 2) % 8 == 0 && (a->o_stride_s * 2) % 8 == 0;
  WC_REQUIRE(al, WC_ERR_ALIGN, "wc_self_attention: x and weight rows need 16-byte, bias and output rows 8-byte "
             "alignment");
  QkvParams p;
  p.nb = static_cast<int>(a->n * a->b);
  p.heads = static_cast<int>(a->heads);
  p.b = static_cast<int>(a->b);
  p.s = static_cast<int>(a->s);
  p.d = static_cast<int>(a->d_model);
  p.scale_log2 = a->scale * 1.4426950408889634f;
  p.x = static_cast<const bf16*>(a->x);
  p.x_sn = a->x_stride_n;
  p.x_sb = a->x_stride_b;
  p.x_ss = a->x_stride_s;
  p.wq = static_cast<const bf16*>(a->q_weight);
  p.wq_sn = a->q_weight_stride_n;
  p.wkv = static_cast<const bf16*>(a->kv_weight);
  p.wkv_sn = a->kv_weight_stride_n;
  p.bq = static_cast<const bf16*>(a->q_bias);
  p.bq_sn = a->q_bias_stride_n;
  p.bkv = static_cast<const bf16*>(a->kv_bias);
  p.bkv_sn = a->kv_bias_stride_n;
  p.o = static_cast<bf16*>(a->o);
  p.o_sb = a->o_stride_nb;
  p.o_ss = a->o_stride_s;
  return a->s > 256 ? launch_qkv<8>(p, a->causal != 0, as_stream(stream))
                    : launch_qkv<4>(p, a->causal != 0, as_stream(stream));
}
