// Grouped (per-model) GEMM on MFMA with a fused bias / residual / ReLU
// epilogue:
//   C[i][m][o] = act( sum_k A[i][m][k] * W[i][o][k] + bias[i][o] + R[i][m][o] )
// A and W are K-contiguous ("NT"), which is exactly the operand layout MFMA
// wants: every lane feeds 8 consecutive k values of one row.
//
// Tiling: a workgroup of WM x WN waves computes a (WM*TM) x (WN*TN) tile of C;
// each wave owns a TM x TN sub-tile made of 16x16 MFMA tiles accumulated in
// fp32.  K advances in steps of 32.  A and W tiles are staged in LDS (double
// buffered: the next K-step is fetched into registers while the current one
// feeds the MFMAs); rows are padded by 16 bytes so the 16-byte fragment reads
// of a quarter-wave hit 64 distinct banks.
//
// bf16 uses v_mfma_f32_16x16x32_bf16 (one instruction per K-step of 32);
// fp32 uses v_mfma_f32_16x16x4_f32 with the K-step permuted so that lane
// group g (lanes 16g..16g+15) contributes k = 8g .. 8g+7 over eight
// instructions -- a reordering of the k summation only.
//
// Rows of A / C may be addressed through a two-level decomposition
// m = outer * rows_inner + inner, so strided N-first views (e.g. the
// channel-packed boundary layout, or [N,B,T,I] inputs) are read in place.
#include "wc_gemm.h"

#include <type_traits>

namespace wc {


namespace {

constexpr int kBK = 32;

template <typename TA> struct Frag;
template <> struct Frag<bf16> { typedef bf16x8 type; };
template <> struct Frag<float> { typedef f32x4 type; };  // two per K-step
template <> struct Frag<f16> { typedef bf16x8 type; };    // raw 16-bit lanes, as bf16


__device__ __forceinline__ float relu_f(float v) { return v > 0.f ? v : 0.f; }

template <typename TA, typename TC, typename TB, int TM, int TN, int WM, int WN, bool VEC>
__global__ __launch_bounds__(WM* WN * 64) void gemm_kernel(GemmParams p) {
  constexpr int NT = WM * WN * 64;
  constexpr int BM = WM * TM, BN = WN * TN;
  constexpr int ES = sizeof(TA);
  constexpr int VE = 16 / ES;                 // elements per 16-byte vector
  constexpr int PITCH = kBK + VE;             // padded LDS row (elements)
  constexpr int CPR = kBK / VE;               // 16-byte chunks per tile row
  constexpr int A_CH = BM * CPR, B_CH = BN * CPR;
  constexpr int A_PT = (A_CH + NT - 1) / NT, B_PT = (B_CH + NT - 1) / NT;
  constexpr int FM = TM / 16, FN = TN / 16;

  __shared__ __attribute__((aligned(16))) TA As[2][BM * PITCH];
  __shared__ __attribute__((aligned(16))) TA Bs[2][BN * PITCH];

  // ---- tile coordinates (XCD-aware: neighbouring tiles share an L2) ----
  const int tiles_per_model = p.tiles_m * p.tiles_o;
  const int nblk = p.n * tiles_per_model;
  int bid = blockIdx.x;
  if (p.remap) bid = (blockIdx.x & 7) * (nblk >> 3) + (blockIdx.x >> 3);
  const int mdl = bid / tiles_per_model;
  const int rem = bid - mdl * tiles_per_model;
  const int to = rem / p.tiles_m;
  const int tm = rem - to * p.tiles_m;
  const int m0 = tm * BM, o0 = to * BN;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave / WN, wn = wave - (wave / WN) * WN;

  const TA* abase = static_cast<const TA*>(p.a) + static_cast<int64_t>(mdl) * p.a_sn;
  const TA* wbase = static_cast<const TA*>(p.w) + static_cast<int64_t>(mdl) * p.w_sn;

  // per-thread global row pointers of the chunks it stages (fixed over K)
  const TA* arow[A_PT];
  int acol[A_PT], aslot[A_PT];
#pragma unroll
  for (int q = 0; q < A_PT; ++q) {
    const int ch = tid + q * NT;
    const int r = ch / CPR;
    acol[q] = (ch - r * CPR) * VE;
    aslot[q] = (ch < A_CH) ? r * PITCH + acol[q] : -1;
    const int gm = m0 + r;
    arow[q] = nullptr;
    if (ch < A_CH && gm < p.m) {
      const uint32_t outer = fdiv(static_cast<uint32_t>(gm), p.a_ri);
      const uint32_t inner = gm - outer * p.a_ri.d;
      arow[q] = abase + static_cast<int64_t>(outer) * p.a_so + static_cast<int64_t>(inner) * p.a_si;
    }
  }
  const TA* brow[B_PT];
  int bcol[B_PT], bslot[B_PT];
#pragma unroll
  for (int q = 0; q < B_PT; ++q) {
    const int ch = tid + q * NT;
    const int r = ch / CPR;
    bcol[q] = (ch - r * CPR) * VE;
    bslot[q] = (ch < B_CH) ? r * PITCH + bcol[q] : -1;
    const int go = o0 + r;
    brow[q] = (ch < B_CH && go < p.o) ? wbase + static_cast<int64_t>(go) * p.k : nullptr;
  }

  uint4 areg[A_PT], breg[B_PT];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int q = 0; q < A_PT; ++q) {
      const int kk = k0 + acol[q];
      if (VEC) {
        areg[q] = (arow[q] && kk < p.k) ? *reinterpret_cast<const uint4*>(arow[q] + kk)
                                        : make_uint4(0, 0, 0, 0);
      } else {
        TA tmp[VE];
#pragma unroll
        for (int e = 0; e < VE; ++e)
          tmp[e] = (arow[q] && kk + e < p.k) ? arow[q][kk + e] : from_f32<TA>(0.f);
        areg[q] = *reinterpret_cast<uint4*>(tmp);
      }
    }
#pragma unroll
    for (int q = 0; q < B_PT; ++q) {
      const int kk = k0 + bcol[q];
      if (VEC) {
        breg[q] = (brow[q] && kk < p.k) ? *reinterpret_cast<const uint4*>(brow[q] + kk)
                                        : make_uint4(0, 0, 0, 0);
      } else {
        TA tmp[VE];
#pragma unroll
        for (int e = 0; e < VE; ++e)
          tmp[e] = (brow[q] && kk + e < p.k) ? brow[q][kk + e] : from_f32<TA>(0.f);
        breg[q] = *reinterpret_cast<uint4*>(tmp);
      }
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int q = 0; q < A_PT; ++q)
      if (aslot[q] >= 0) *reinterpret_cast<uint4*>(&As[buf][aslot[q]]) = areg[q];
#pragma unroll
    for (int q = 0; q < B_PT; ++q)
      if (bslot[q] >= 0) *reinterpret_cast<uint4*>(&Bs[buf][bslot[q]]) = breg[q];
  };

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int ktiles = (p.k + kBK - 1) / kBK;
  fetch(0);
  stash(0);
  __syncthreads();

  const int fr = lane & 15;          // fragment row / column
  const int fk = (lane >> 4) * 8;    // first k of this lane group
  for (int kt = 0; kt < ktiles; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < ktiles) fetch((kt + 1) * kBK);
    const TA* as = As[buf];
    const TA* bs = Bs[buf];
    if constexpr (sizeof(TA) == 2) {
      bf16x8 af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(&as[(wm * TM + i * 16 + fr) * PITCH + fk]);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8*>(&bs[(wn * TN + j * 16 + fr) * PITCH + fk]);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = mma16<TA>(af[i], bfr[j], acc[i][j]);
    } else {
      f32x4 af[FM][2], bfr[FN][2];
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const float* src = reinterpret_cast<const float*>(&as[(wm * TM + i * 16 + fr) * PITCH + fk]);
        af[i][0] = *reinterpret_cast<const f32x4*>(src);
        af[i][1] = *reinterpret_cast<const f32x4*>(src + 4);
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const float* src = reinterpret_cast<const float*>(&bs[(wn * TN + j * 16 + fr) * PITCH + fk]);
        bfr[j][0] = *reinterpret_cast<const f32x4*>(src);
        bfr[j][1] = *reinterpret_cast<const f32x4*>(src + 4);
      }
#pragma unroll
      for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][s >> 2][s & 3], bfr[j][s >> 2][s & 3],
                                                             acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < ktiles) {
      stash(buf ^ 1);
      __syncthreads();
    }
  }

  // ---- epilogue: bias, residual, activation, store ----
  const TB* bias = p.bias ? static_cast<const TB*>(p.bias) + static_cast<int64_t>(mdl) * p.b_sn : nullptr;
  TC* cbase = static_cast<TC*>(p.c) + static_cast<int64_t>(mdl) * p.c_sn;
  const TC* rbase = p.r ? static_cast<const TC*>(p.r) + static_cast<int64_t>(mdl) * p.r_sn : nullptr;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int col = o0 + wn * TN + j * 16 + fr;
    if (col >= p.o) continue;
    const float bv = bias ? to_f32(bias[col]) : 0.f;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = m0 + wm * TM + i * 16 + (lane >> 4) * 4 + e;
        if (row >= p.m) continue;
        const uint32_t outer = fdiv(static_cast<uint32_t>(row), p.c_ri);
        const uint32_t inner = row - outer * p.c_ri.d;
        const int64_t off = static_cast<int64_t>(outer) * p.c_so + static_cast<int64_t>(inner) * p.c_si + col;
        float v = acc[i][j][e] + bv;
        if (rbase) {
          const int64_t roff = static_cast<int64_t>(outer) * p.r_so + static_cast<int64_t>(inner) * p.r_si + col;
          v += to_f32(rbase[roff]);
        }
        if (p.act == WC_ACT_RELU) v = relu_f(v);
        cbase[off] = from_f32<TC>(v);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Large-tile bf16 kernel.  A workgroup of WM x WN waves computes a
// (WM*FM*16) x (WN*FN*16) tile; K advances in tiles of 64 staged through a
// double-buffered LDS ring (each thread moves 16-byte chunks global ->
// registers -> LDS; the next tile's loads are in flight during the current
// tile's 2 x FM x FN MFMAs).  The epilogue goes through LDS as well: each wave
// parks a 16-row strip of its fp32 accumulators, reads it back row-major and
// applies bias / residual / ReLU with 8- or 16-byte stores along rows.
// ---------------------------------------------------------------------------
constexpr int kBigBK = 64;
constexpr int kBigPitch = kBigBK + 8;          // bf16 elements per LDS row (144 bytes)

template <int WM, int WN, int FM, int FN>
struct BigCfg {
  static constexpr int NT = WM * WN * 64;
  static constexpr int BM = WM * FM * 16, BN = WN * FN * 16;
  static constexpr int CH = (BM + BN) * (kBigBK / 8);        // 16-byte chunks per stage
  static constexpr int CPT = CH / NT;                       // chunks per thread
  static constexpr int STAGE = (BM + BN) * kBigPitch;       // bf16 elements per stage
  static constexpr int EPI_PITCH = FN * 16 + 4;             // floats per epilogue row
  static constexpr size_t LDS_MAIN = 2 * STAGE * sizeof(bf16);
  static constexpr size_t LDS_EPI = static_cast<size_t>(WM * WN) * 16 * EPI_PITCH * sizeof(float);
  static constexpr size_t LDS = LDS_MAIN > LDS_EPI ? LDS_MAIN : LDS_EPI;
  static_assert(CH % NT == 0, "chunks must divide evenly");
};

template <typename TA, typename TC, typename TB, int WM, int WN, int FM, int FN>
__global__ __launch_bounds__(WM* WN * 64) void gemm_big_kernel(GemmParams p) {
  using C = BigCfg<WM, WN, FM, FN>;
  constexpr int NT = C::NT, BM = C::BM, BN = C::BN, CPT = C::CPT;
  extern __shared__ __attribute__((aligned(16))) bf16 big_smem[];

  const int tiles_per_model = p.tiles_m * p.tiles_o;
  const int nblk = p.n * tiles_per_model;
  int bid = blockIdx.x;
  if (p.remap) bid = (blockIdx.x & 7) * (nblk >> 3) + (blockIdx.x >> 3);
  const int mdl = bid / tiles_per_model;
  const int rem = bid - mdl * tiles_per_model;
  const int to = rem / p.tiles_m;
  const int tm = rem - to * p.tiles_m;
  const int m0 = tm * BM, o0 = to * BN;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave / WN, wn = wave - (wave / WN) * WN;

  const bf16* abase = static_cast<const bf16*>(p.a) + static_cast<int64_t>(mdl) * p.a_sn;
  const bf16* wbase = static_cast<const bf16*>(p.w) + static_cast<int64_t>(mdl) * p.w_sn;

  // staging: chunk c = tid + q*NT; rows [0, BM) are A, [BM, BM+BN) are W
  const bf16* src[CPT];
  int dst[CPT];
#pragma unroll
  for (int q = 0; q < CPT; ++q) {
    const int c = tid + q * NT;
    const int r = c >> 3, kc = (c & 7) * 8;
    dst[q] = r * kBigPitch + kc;
    src[q] = nullptr;
    if (r < BM) {
      const int gm = m0 + r;
      if (gm < p.m) {
        const uint32_t outer = fdiv(static_cast<uint32_t>(gm), p.a_ri);
        const uint32_t inner = gm - outer * p.a_ri.d;
        src[q] = abase + static_cast<int64_t>(outer) * p.a_so + static_cast<int64_t>(inner) * p.a_si + kc;
      }
    } else {
      const int go = o0 + (r - BM);
      if (go < p.o) src[q] = wbase + static_cast<int64_t>(go) * p.k + kc;
    }
  }
  uint4 stg[CPT];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int q = 0; q < CPT; ++q) {
      const int kk = k0 + (dst[q] % kBigPitch);
      stg[q] = (src[q] && kk < p.k) ? *reinterpret_cast<const uint4*>(src[q] + k0) : make_uint4(0, 0, 0, 0);
    }
  };
  auto stash = [&](int stage) {
    bf16* base = big_smem + stage * C::STAGE;
#pragma unroll
    for (int q = 0; q < CPT; ++q) *reinterpret_cast<uint4*>(base + dst[q]) = stg[q];
  };

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int ktiles = (p.k + kBigBK - 1) / kBigBK;
  fetch(0);
  stash(0);
  __syncthreads();
  const int fr = lane & 15, fk = (lane >> 4) * 8;
  for (int kt = 0; kt < ktiles; ++kt) {
    const int stage = kt & 1;
    if (kt + 1 < ktiles) fetch((kt + 1) * kBigBK);
    const bf16* as = big_smem + stage * C::STAGE + (wm * FM * 16 + fr) * kBigPitch + fk;
    const bf16* bs = big_smem + stage * C::STAGE + (BM + wn * FN * 16 + fr) * kBigPitch + fk;
#pragma unroll
    for (int kk = 0; kk < kBigBK; kk += 32) {
      bf16x8 af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) af[i] = *reinterpret_cast<const bf16x8*>(as + i * 16 * kBigPitch + kk);
#pragma unroll
      for (int j = 0; j < FN; ++j) bfr[j] = *reinterpret_cast<const bf16x8*>(bs + j * 16 * kBigPitch + kk);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = mma16<TA>(af[i], bfr[j], acc[i][j]);
    }
    if (kt + 1 < ktiles) stash(stage ^ 1);
    __syncthreads();
  }

  // ---- epilogue through LDS: one 16-row strip of the wave's tile at a time ----
  constexpr int EP = C::EPI_PITCH;
  constexpr int COLS = FN * 16;
  constexpr int LPR = COLS / 4;                  // lanes per row (4 columns each)
  constexpr int RPI = 64 / LPR;                  // rows per read instruction
  float* ep = reinterpret_cast<float*>(big_smem) + wave * 16 * EP;
  const TB* bias = p.bias ? static_cast<const TB*>(p.bias) + static_cast<int64_t>(mdl) * p.b_sn : nullptr;
  TC* cbase = static_cast<TC*>(p.c) + static_cast<int64_t>(mdl) * p.c_sn;
  const TC* rbase = p.r ? static_cast<const TC*>(p.r) + static_cast<int64_t>(mdl) * p.r_sn : nullptr;
  const int lc = (lane % LPR) * 4;               // this lane's 4 columns within the strip
  const int col0 = o0 + wn * COLS + lc;
  const bool vec4 = (p.o & 3) == 0;
  float bv[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) bv[e] = (bias && col0 + e < p.o) ? to_f32(bias[col0 + e]) : 0.f;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) ep[((lane >> 4) * 4 + e) * EP + j * 16 + fr] = acc[i][j][e];
    __builtin_amdgcn_s_waitcnt(0xc07f);          // lgkmcnt(0): this wave's strip is in LDS
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int rr = 0; rr < 16; rr += RPI) {
      const int lr = rr + lane / LPR;
      const int row = m0 + wm * FM * 16 + i * 16 + lr;
      const f32x4 v4 = *reinterpret_cast<const f32x4*>(ep + lr * EP + lc);
      if (row < p.m && col0 < p.o) {
        const uint32_t outer = fdiv(static_cast<uint32_t>(row), p.c_ri);
        const uint32_t inner = row - outer * p.c_ri.d;
        const int64_t off = static_cast<int64_t>(outer) * p.c_so + static_cast<int64_t>(inner) * p.c_si + col0;
        float v[4] = {v4[0] + bv[0], v4[1] + bv[1], v4[2] + bv[2], v4[3] + bv[3]};
        if (rbase) {
          const int64_t roff = static_cast<int64_t>(outer) * p.r_so + static_cast<int64_t>(inner) * p.r_si + col0;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (col0 + e < p.o) v[e] += to_f32(rbase[roff + e]);
        }
        if (p.act == WC_ACT_RELU)
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = relu_f(v[e]);
        if (vec4 && col0 + 3 < p.o) {
          if constexpr (sizeof(TC) == 4) {
            *reinterpret_cast<f32x4*>(cbase + off) = f32x4{v[0], v[1], v[2], v[3]};
          } else {
            typedef TC tc4 __attribute__((ext_vector_type(4)));
            tc4 o4;
#pragma unroll
            for (int e = 0; e < 4; ++e) o4[e] = from_f32<TC>(v[e]);
            *reinterpret_cast<tc4*>(cbase + off) = o4;
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (col0 + e < p.o) cbase[off + e] = from_f32<TC>(v[e]);
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
  }
}

// ---------------------------------------------------------------------------
// Persistent XL bf16 kernel (bf16 output).  Requires K % 64 == 0, M, O and
// both row decompositions' rows_inner % 16 == 0, 16-byte aligned output /
// residual rows and per-model byte offsets below 2^31 (checked on the host).
//
// One workgroup per CU walks a list of 256 x 256 output tiles; the tiles of
// one XCD (workgroup index % 8) form a contiguous range of the (model, column
// tile, row tile) order, so the 32 CUs sharing an L2 work on neighbouring
// tiles: the same activation rows and a few weight tiles.  4 waves in 2 x 2,
// each 128 x 128 as 8 x 8 MFMA 16x16x32 tiles (one wave per SIMD, the 256
// accumulators per lane in AGPRs).  MFMA roles are swapped with respect to C:
// the A operand is a W row (o), the B operand an activation row (m), so a
// lane's 4 accumulators are 4 consecutive output columns of one row.  The
// accumulators of a tile start at zero (the first MFMA takes a zero C operand)
// and the epilogue adds the bias.
//
// K advances in stages of 64 (128-byte row segments: whole cache lines)
// through 2 LDS slots of 64 KB, in a rotated order per tile (see tile_of); the
// stage sequence runs on across tile boundaries, so the next tile's operands
// load during the current tile's last stage and epilogue.  Operands move
// global -> LDS with
// global_load_lds_dwordx4: one instruction moves 8 rows x 128 bytes into a
// contiguous 1 KB; the 16-byte chunk c of row r sits at position c ^ (r & 7),
// so the 8 rows a fragment read serves per pass hit 8 distinct bank groups.
// Fragments are double-buffered in registers per 32-wide half stage: the
// second half's fragments are read during the first half's MFMAs, and the
// next stage's first half during the second half's.  Past the last stage the
// ring is fed copies of the last stage (into the free slot), so the stage
// loop has no branches.  Barriers are bare s_barrier with explicit waits: a
// workgroup fence would also wait for the loads in flight.
//
// Epilogue: stores and residual loads are buffer operations whose
// out-of-range lanes the hardware drops, and the next tile's bias loads are
// issued there too, so every wave issues a fixed number of memory
// instructions per tile and the vmcnt waits stay exact.
// ---------------------------------------------------------------------------
constexpr int kXlB = 256, kXlBK = 64, kXlThreads = 256;
constexpr int kXlHalf = kXlB * kXlBK * 2;                 // bytes of one operand per stage (32 KB)
constexpr int kXlStageBytes = 2 * kXlHalf;                // 64 KB
constexpr int kXlStripPitch = 128 * 2 + 16;               // bf16 epilogue strip row (bytes)
constexpr int kXlStripBytes = 16 * kXlStripPitch;         // per wave
constexpr uint32_t kXlOob = 0x80000000u;                  // buffer offset of a dropped lane

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __attribute__((address_space(3))) char lds_char;
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
typedef __attribute__((address_space(3))) i32x4 lds_i32x4;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t xl_rsrc(const void* base, int32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// VMEM instructions one wave issues per tile epilogue: 32 stores (+ 32 residual
// loads) and the LDS-DMA load of its quarter of the next tile's bias.
template <bool RES>
struct XlEpi {
  static constexpr int value = 32 * (RES ? 2 : 1) + 1;
};
constexpr int kXlBiasSlot = kXlB * 4;                     // bytes of one tile's bias (fp32 at most)

// s_waitcnt vmcnt(N) lgkmcnt(0) (gfx9 encoding: vmcnt in bits 3:0 and 15:14,
// expcnt 6:4 left at 7, lgkmcnt 11:8)
template <int N>
__device__ __forceinline__ void vm_lgkm_wait() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4));
}

// Workgroup barrier without a memory fence: the caller has already waited
// for what the other waves must see.  The empty asm statements keep the
// compiler from moving memory accesses across it.
__device__ __forceinline__ void bare_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// One LDS-DMA instruction of a stage: block q < 8 moves W rows r0 + 64 wave + 8 q,
// block q >= 8 A rows r0 + 64 wave + 8 (q - 8) (r0 = the tile's first column / row),
// 128 bytes of K each, into the stage slot at `st`.  Blocks past the last row
// reload the last 8 rows (their results are never stored).
__device__ __forceinline__ void xl_dma_block(const GemmParams& p, const char* wmod, const char* amod, lds_char* st,
                                             int r0, int wave, int q, uint32_t wlane, uint32_t alane) {
  if (q < 8) {
    const int rb = min(r0 + 64 * wave + 8 * q, p.o - 8);
    __builtin_amdgcn_global_load_lds(wmod + static_cast<uint32_t>(rb) * static_cast<uint32_t>(p.k) * 2u + wlane,
                                     (lds_ptr_t)(st + (64 * wave + 8 * q) * 128), 16, 0, 0);
  } else {
    const int rb = min(r0 + 64 * wave + 8 * (q - 8), p.m - 8);
    const uint32_t outer = fdiv(static_cast<uint32_t>(rb), p.a_ri);
    const uint32_t inner = rb - outer * p.a_ri.d;
    const uint32_t off = (outer * static_cast<uint32_t>(p.a_so) + inner * static_cast<uint32_t>(p.a_si)) * 2u;
    __builtin_amdgcn_global_load_lds(amod + off + alane, (lds_ptr_t)(st + kXlHalf + (64 * wave + 8 * (q - 8)) * 128),
                                     16, 0, 0);
  }
}

template <typename TA, typename TB, bool RES, bool RELU>
__global__ __launch_bounds__(kXlThreads, 1) void gemm_xlp_kernel(GemmParams p, int tiles_total) {
  __shared__ __attribute__((aligned(1024))) char smem_raw[2 * kXlStageBytes + 4 * kXlStripBytes + 2 * kXlBiasSlot];
  lds_char* const smem = (lds_char*)smem_raw;        // keeps every LDS address 32-bit
  constexpr int E = XlEpi<RES>::value;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int ow = (wave & 1) * 128, mw = (wave >> 1) * 128;
  const int tiles_per_model = p.tiles_m * p.tiles_o;
  const int KS = p.k / kXlBK;

  // ---- this workgroup's tiles: XCD x = blockIdx % 8 owns a contiguous range ----
  const int G = gridDim.x;
  int t_first, t_step, my_tiles;
  if ((G & 7) == 0) {
    const int x = blockIdx.x & 7, l = blockIdx.x >> 3, nwx = G >> 3;
    const int lo = static_cast<int>((static_cast<int64_t>(tiles_total) * x) >> 3);
    const int hi = static_cast<int>((static_cast<int64_t>(tiles_total) * (x + 1)) >> 3);
    t_first = lo + l;
    t_step = nwx;
    my_tiles = t_first < hi ? (hi - t_first + nwx - 1) / nwx : 0;
  } else {
    t_first = blockIdx.x;
    t_step = G;
    my_tiles = t_first < tiles_total ? (tiles_total - t_first + G - 1) / G : 0;
  }
  const int S = my_tiles * KS;
  if (S == 0) return;

  // A tile's K stages run in a rotated order, starting at stage (m-tile index mod
  // KS): the workgroups that share a block of W rows (same model and column tile,
  // consecutive m tiles, resident on one XCD at the same time) then read different
  // K slices of it at any moment, and only the first to reach a slice misses in L2.
  struct Tile { int mdl, m0, o0, rot; };
  auto tile_of = [&](int ti) {
    Tile t;
    const int g = t_first + ti * t_step;
    t.mdl = static_cast<int>(fdiv(static_cast<uint32_t>(g), p.fd_tpm));
    const int rem = g - t.mdl * tiles_per_model;
    const int to = static_cast<int>(fdiv(static_cast<uint32_t>(rem), p.fd_tm));
    const int mt = rem - to * p.tiles_m;
    t.m0 = mt * kXlB;
    t.o0 = to * kXlB;
    t.rot = mt - static_cast<int>(fdiv(static_cast<uint32_t>(mt), p.fd_ks)) * KS;
    return t;
  };

  // ---- DMA of stage `stage` into slot stage & 1 (stages past the last reload it) ----
  // Lane l of an 8-row block instruction writes LDS bytes [16 l, 16 l + 16): row
  // l >> 3, position l & 7, which receives global chunk (l & 7) ^ (l >> 3).
  // Block q < 8 is W rows o0 + 64 wave + 8 q, block q >= 8 A rows m0 + 64 wave + 8 (q - 8).
  const uint32_t dchunk = ((lane & 7) ^ (lane >> 3)) * 8;
  const uint32_t wlane = ((lane >> 3) * static_cast<uint32_t>(p.k) + dchunk) * 2u;
  const uint32_t alane = ((lane >> 3) * static_cast<uint32_t>(p.a_si) + dchunk) * 2u;
  // DMA source of stage `stage`: model bases of W and A at the stage's (rotated) K
  // slice, and the tile's first rows
  struct Dma { const char* wmod; const char* amod; int slot, o0, m0; };
  auto dma_of = [&](int stage) {
    const int sidx = stage < S ? stage : S - 1;
    const int ti = static_cast<int>(fdiv(static_cast<uint32_t>(sidx), p.fd_ks));
    const Tile t = tile_of(ti);
    int ks = sidx - ti * KS + t.rot;
    if (ks >= KS) ks -= KS;
    Dma d;
    d.wmod = static_cast<const char*>(p.w) + static_cast<int64_t>(t.mdl) * p.w_sn * 2 + ks * 128;
    d.amod = static_cast<const char*>(p.a) + static_cast<int64_t>(t.mdl) * p.a_sn * 2 + ks * 128;
    d.slot = (stage & 1) * kXlStageBytes;
    d.o0 = t.o0;
    d.m0 = t.m0;
    return d;
  };
  auto dma_block = [&](const Dma& d, int q) {
    xl_dma_block(p, d.wmod, d.amod, smem + d.slot, q < 8 ? d.o0 : d.m0, wave, q, wlane, alane);
  };
  auto issue = [&](int stage) {
    const Dma d = dma_of(stage);
#pragma unroll
    for (int q = 0; q < 16; ++q) dma_block(d, q);
  };

  // fragment byte offsets: row = base + 16 * i + (lane & 15), chunk 4 * half + (lane >> 4)
  const int fr = lane & 15;
  const int fp0 = (((lane >> 4)) ^ (fr & 7)) << 4;
  const int fp1 = ((4 + (lane >> 4)) ^ (fr & 7)) << 4;
  const int wfo = (ow + fr) * 128, afo = kXlHalf + (mw + fr) * 128;
  // fragment g of a K half: g < 8 is W rows ow + 16 g, g >= 8 A rows mw + 16 (g - 8)
  auto read_frag = [&](int stage, int fpos, int g, bf16x8 (&wf)[8], bf16x8 (&af)[8]) {
    const lds_char* st = smem + (stage & 1) * kXlStageBytes + fpos;
    if (g < 8)
      wf[g] = *(const lds_bf16x8*)(st + wfo + g * 2048);
    else
      af[g - 8] = *(const lds_bf16x8*)(st + afo + (g - 8) * 2048);
  };
  auto read_frags = [&](int stage, int fpos, bf16x8 (&wf)[8], bf16x8 (&af)[8]) {
#pragma unroll
    for (int g = 0; g < 16; ++g) read_frag(stage, fpos, g, wf, af);
  };

  // ---- bias of a tile: wave w moves the tile's columns [64 w, 64 w + 64) into LDS slot
  // (tile index & 1) with one LDS-DMA load (columns past o read a valid column; the
  // stores of those columns are dropped).  The epilogue adds it; the accumulators of
  // a tile start at zero (the first MFMA of each takes a zero C operand). ----
  lds_char* const bias_lds = smem + 2 * kXlStageBytes + 4 * kXlStripBytes;
  // The lane index, recomputed (v_mbcnt) where it is needed outside the stage loop: a
  // lane-derived value kept live across the loop gets spilled, and a spill reload's
  // vmcnt wait would also wait for the operand loads of the next stages.
  auto lane_now = []() {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
  };
  const char* const bias_base = p.bias ? static_cast<const char*>(p.bias) : static_cast<const char*>(p.c);
  auto load_bias = [&](const Tile& t, int slot) {
    constexpr int EPC = 16 / static_cast<int>(sizeof(TB));       // bias elements per 16-byte chunk
    constexpr int LANES = 64 / EPC;                               // lanes that move the wave's 64 columns
    const int lane = lane_now();
    const int col = t.o0 + 64 * wave + EPC * (lane < LANES ? lane : 0);
    const int cl = col < p.o ? col : p.o - EPC;
    const int64_t eoff = p.bias ? static_cast<int64_t>(t.mdl) * p.b_sn + cl : 0;
    if (lane < LANES)
      __builtin_amdgcn_global_load_lds(bias_base + eoff * static_cast<int64_t>(sizeof(TB)),
                                       (lds_ptr_t)(bias_lds + slot * kXlBiasSlot + 64 * wave * sizeof(TB)), 16, 0, 0);
  };

  f32x4 acc[8][8];

  // ---- epilogue of tile t: acc (+residual, ReLU) -> C, one 16-row strip at a time
  // through LDS, then 16-byte row chunks: lane -> row 4 q + (lane >> 4), 8 columns
  // from 8 (lane & 15) ----
  lds_char* strip = smem + 2 * kXlStageBytes + wave * kXlStripBytes;
  auto epilogue = [&](const Tile& t, int ti_parity) {
    const __amdgpu_buffer_rsrc_t crs =
        xl_rsrc(static_cast<TA*>(p.c) + static_cast<int64_t>(t.mdl) * p.c_sn, p.c_bytes);
    const __amdgpu_buffer_rsrc_t rrs =
        xl_rsrc(RES ? static_cast<const TA*>(p.r) + static_cast<int64_t>(t.mdl) * p.r_sn : p.c, p.r_bytes);
    constexpr bool relu = RELU;
    const int lane = lane_now();
    const int fr = lane & 15;
    // bias of the lane's columns ow + 16 i + 4 (lane >> 4) + e.  With one stage per
    // tile no stage wait has covered the bias load issued after the previous epilogue.
    if (KS == 1) {
      vm_lgkm_wait<0>();
      bare_barrier();
    }
    float bv[8][4];
    {
      const lds_char* bl = bias_lds + (ti_parity & 1) * kXlBiasSlot + (ow + 4 * (lane >> 4)) * sizeof(TB);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if constexpr (sizeof(TB) == 4) {
          const f32x4 b4 = *(const __attribute__((address_space(3))) f32x4*)(bl + 16 * i * 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) bv[i][e] = p.bias ? b4[e] : 0.f;
        } else {
          typedef TB tb4 __attribute__((ext_vector_type(4)));
          typedef __attribute__((address_space(3))) tb4 lds_tb4;
          const auto b4 = *(const lds_tb4*)(bl + 16 * i * 2);
#pragma unroll
          for (int e = 0; e < 4; ++e) bv[i][e] = p.bias ? to_f32(b4[e]) : 0.f;
        }
      }
    }
    const int cc = lane & 15, rsub = lane >> 4;
    const int col = t.o0 + ow + cc * 8;
    const bool col_ok = col < p.o;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        bf16x4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float v = acc[i][j][e] + bv[i][e];
          if (!RES && relu) v = relu_f(v);
          o4[e] = __builtin_bit_cast(bf16, from_f32<TA>(v));   // the strip holds raw 16-bit values
        }
        *(lds_bf16x4*)(strip + fr * kXlStripPitch + (16 * i + 4 * (lane >> 4)) * 2) = o4;
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);          // lgkmcnt(0): strip written
      __builtin_amdgcn_wave_barrier();
      // the strip's 16 rows share one row decomposition (rows_inner % 16 == 0)
      const int row0 = t.m0 + mw + 16 * j;
      const uint32_t outer = fdiv(static_cast<uint32_t>(row0), p.c_ri);
      const uint32_t inner = row0 - outer * p.c_ri.d;
      const bool strip_ok = row0 < p.m && col_ok;
      const uint32_t cbase = (outer * static_cast<uint32_t>(p.c_so) + inner * static_cast<uint32_t>(p.c_si) + col) * 2u;
      const uint32_t rbase = (outer * static_cast<uint32_t>(p.r_so) + inner * static_cast<uint32_t>(p.r_si) + col) * 2u;
      i32x4 raw[4], rv[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int lr = 4 * q + rsub;
        raw[q] = *(const lds_i32x4*)(strip + lr * kXlStripPitch + cc * 16);
        if constexpr (RES)
          rv[q] = __builtin_amdgcn_raw_buffer_load_b128(
              rrs, strip_ok ? rbase + static_cast<uint32_t>(lr * p.r_si) * 2u : kXlOob, 0, 0);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int lr = 4 * q + rsub;
        i32x4 outv = raw[q];
        if constexpr (RES) {
          const TA* a = reinterpret_cast<const TA*>(&raw[q]);
          const TA* b = reinterpret_cast<const TA*>(&rv[q]);
          TA* o = reinterpret_cast<TA*>(&outv);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            float v = to_f32(a[e]) + to_f32(b[e]);
            if (relu) v = relu_f(v);
            o[e] = from_f32<TA>(v);
          }
        }
        // non-temporal (nt): the output streams past the L2s, which keep the operand tiles
        __builtin_amdgcn_raw_buffer_store_b128(
            outv, crs, strip_ok ? cbase + static_cast<uint32_t>(lr * p.c_si) * 2u : kXlOob, 0, 2);
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);          // strip reads done before it is rewritten
      __builtin_amdgcn_wave_barrier();
    }
  };

  // ---- prologue: stage 0 landed and its first half read, stage 1 in flight ----
  issue(0);
  load_bias(tile_of(0), 0);
  vm_lgkm_wait<0>();
  bare_barrier();
  issue(1);
  bf16x8 w0[8], a0[8], w1[8], a1[8];
  read_frags(0, fp0, w0, a0);

  auto mfma_half = [&](bf16x8 (&wf)[8], bf16x8 (&af)[8], auto first_tag) {
    constexpr bool kFirst = decltype(first_tag)::value;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[i][j] = mma16<TA>(wf[i], af[j], kFirst ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[i][j]);
  };
  auto interleave = [&]() {
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);     // one fragment read
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);     // four MFMAs
    }
  };
  // stage s: first half's MFMAs with the second half's fragments read in between;
  // wait for stage s + 1 (behind it only the epilogue of a tile that ended at
  // s - 1), refill slot s & 1 with stage s + 2; second half's MFMAs with stage
  // s + 1's first-half fragments read in between
  //
  // The last stage of a tile does not read the next stage's fragments: they are read
  // after the epilogue, so that 64 fragment registers are free while it runs.
  using yes = std::true_type;
  using no = std::false_type;
  //
  // The 16 DMA instructions of stage s + 2 are spread over the second half's MFMAs
  // (program order DMA g, fragment read g; the scheduler puts two MFMAs between
  // them): issued back to back they stall the wave while the address unit
  // drains them, and no MFMA issues meanwhile.
  auto interleave_dma = [&](auto reads_tag) {
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);     // one DMA
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);     // two MFMAs
      if constexpr (decltype(reads_tag)::value)
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // one fragment read
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);     // two MFMAs
    }
  };
  auto step = [&](bool after_epi, int s, auto first_tag, auto last_tag) {
    constexpr bool kLast = decltype(last_tag)::value;
    read_frags(s, fp1, w1, a1);
    mfma_half(w0, a0, first_tag);
    interleave();
    if (after_epi) vm_lgkm_wait<(E > 63 ? 63 : E)>();
    else vm_lgkm_wait<0>();
    bare_barrier();
    {
      const Dma d = dma_of(s + 2);
#pragma unroll
      for (int g = 0; g < 16; ++g) {
        dma_block(d, g);
        if constexpr (!kLast) read_frag(s + 1, fp0, g, w0, a0);
      }
    }
    mfma_half(w1, a1, no{});
    if constexpr (kLast) interleave_dma(no{});
    else interleave_dma(yes{});
  };
  for (int ti = 0; ti < my_tiles; ++ti) {
    if (KS == 1) {
      step(ti > 0, ti * KS, yes{}, yes{});
    } else {
      step(ti > 0, ti * KS, yes{}, no{});
      for (int ks = 1; ks < KS - 1; ++ks) step(false, ti * KS + ks, no{}, no{});
      step(false, ti * KS + KS - 1, no{}, yes{});
    }
    epilogue(tile_of(ti), ti);
    load_bias(tile_of(ti + 1 < my_tiles ? ti + 1 : ti), (ti + 1) & 1);
    read_frags((ti + 1) * KS, fp0, w0, a0);
  }
}
// ---------------------------------------------------------------------------
// Persistent XL bf16 kernel, two waves per SIMD (bf16 output, no residual).
// The tile walk, the K-stage ring, the LDS layout of a stage and its LDS-DMA
// staging are those of gemm_xlp_kernel; the 256 x 256 tile is split over 8
// waves (2 x 4) of 128 x 64 each, as 8 x 4 MFMA 16x16x32 blocks (128
// accumulators per lane).  Two waves per SIMD keep v_mfma_f32_16x16x32_bf16
// issuing every ~19 cycles where one wave manages ~28.  Wave w moves 4 of a
// stage's W row blocks and 4 of its A row blocks (8 rows x 128 bytes each),
// streams its 8 W and 4 A fragments per 32-wide half stage through registers
// a few MFMA groups ahead of their use (see the main loop), and stores its
// output through a 16-row x 64-column LDS half strip.
// ---------------------------------------------------------------------------
constexpr int kX8Threads = 512;
constexpr int kX8StripPitch = 64 * 2 + 16;                // bf16 half-strip row: 64 columns (bytes)
constexpr int kX8StripBytes = 16 * kX8StripPitch;         // per wave

template <typename TA, typename TB, bool RELU>
__global__ __launch_bounds__(kX8Threads, 1) void gemm_xl8_kernel(GemmParams p, int tiles_total) {
  __shared__ __attribute__((aligned(1024))) char smem_raw[2 * kXlStageBytes + 8 * kX8StripBytes + 2 * kXlBiasSlot];
  lds_char* const smem = (lds_char*)smem_raw;        // keeps every LDS address 32-bit
  // VMEM instructions a wave issues per tile epilogue: 16 stores and its bias load
  constexpr int E = 17;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int ow = (wave & 1) * 128, mw = (wave >> 1) * 64;
  const int tiles_per_model = p.tiles_m * p.tiles_o;
  const int KS = p.k / kXlBK;

  // ---- this workgroup's tiles: XCD x = blockIdx % 8 owns a contiguous range ----
  const int G = gridDim.x;
  int t_first, t_step, my_tiles;
  if ((G & 7) == 0) {
    const int x = blockIdx.x & 7, l = blockIdx.x >> 3, nwx = G >> 3;
    const int lo = static_cast<int>((static_cast<int64_t>(tiles_total) * x) >> 3);
    const int hi = static_cast<int>((static_cast<int64_t>(tiles_total) * (x + 1)) >> 3);
    t_first = lo + l;
    t_step = nwx;
    my_tiles = t_first < hi ? (hi - t_first + nwx - 1) / nwx : 0;
  } else {
    t_first = blockIdx.x;
    t_step = G;
    my_tiles = t_first < tiles_total ? (tiles_total - t_first + G - 1) / G : 0;
  }
  const int S = my_tiles * KS;
  if (S == 0) return;

  // tile ti of this workgroup; its K stages run in a rotated order starting at stage
  // (m-tile index mod KS), as in gemm_xlp_kernel
  struct Tile { int mdl, m0, o0, rot; };
  auto tile_of = [&](int ti) {
    Tile t;
    const int g = t_first + ti * t_step;
    t.mdl = static_cast<int>(fdiv(static_cast<uint32_t>(g), p.fd_tpm));
    const int rem = g - t.mdl * tiles_per_model;
    const int to = static_cast<int>(fdiv(static_cast<uint32_t>(rem), p.fd_tm));
    const int mt = rem - to * p.tiles_m;
    t.m0 = mt * kXlB;
    t.o0 = to * kXlB;
    t.rot = mt - static_cast<int>(fdiv(static_cast<uint32_t>(mt), p.fd_ks)) * KS;
    return t;
  };

  // ---- DMA of stage `stage` into slot stage & 1 (stages past the last reload it).
  // Wave w moves the blocks gemm_xlp_kernel's wave w / 2 moves as its blocks
  // 4 (w & 1) .. + 3 (W rows) and 8 + 4 (w & 1) .. + 3 (A rows): W and A rows
  // 32 w + 8 q' for q' < 4.  Lane l writes row l >> 3 of a block, position l & 7,
  // which receives global chunk (l & 7) ^ (l >> 3). ----
  const uint32_t dchunk = ((lane & 7) ^ (lane >> 3)) * 8;
  const uint32_t wlane = ((lane >> 3) * static_cast<uint32_t>(p.k) + dchunk) * 2u;
  const uint32_t alane = ((lane >> 3) * static_cast<uint32_t>(p.a_si) + dchunk) * 2u;
  struct Dma { const char* wmod; const char* amod; int slot, o0, m0; };
  auto dma_of = [&](int stage) {
    const int sidx = stage < S ? stage : S - 1;
    const int ti = static_cast<int>(fdiv(static_cast<uint32_t>(sidx), p.fd_ks));
    const Tile t = tile_of(ti);
    int ks = sidx - ti * KS + t.rot;
    if (ks >= KS) ks -= KS;
    Dma d;
    d.wmod = static_cast<const char*>(p.w) + static_cast<int64_t>(t.mdl) * p.w_sn * 2 + ks * 128;
    d.amod = static_cast<const char*>(p.a) + static_cast<int64_t>(t.mdl) * p.a_sn * 2 + ks * 128;
    d.slot = (stage & 1) * kXlStageBytes;
    d.o0 = t.o0;
    d.m0 = t.m0;
    return d;
  };
  // block q (0..7) of this wave: q < 4 W rows, q >= 4 A rows
  auto dma_block = [&](const Dma& d, int q) {
    const int qq = q < 4 ? 4 * (wave & 1) + q : 8 + 4 * (wave & 1) + (q - 4);
    xl_dma_block(p, d.wmod, d.amod, smem + d.slot, q < 4 ? d.o0 : d.m0, wave >> 1, qq, wlane, alane);
  };
  auto issue = [&](int stage) {
    const Dma d = dma_of(stage);
#pragma unroll
    for (int q = 0; q < 8; ++q) dma_block(d, q);
  };

  // fragment byte offsets: row = base + 16 * i + (lane & 15), chunk 4 * half + (lane >> 4)
  const int fr = lane & 15;
  const int fp0 = (((lane >> 4)) ^ (fr & 7)) << 4;
  const int fp1 = ((4 + (lane >> 4)) ^ (fr & 7)) << 4;
  const int wfo = (ow + fr) * 128, afo = kXlHalf + (mw + fr) * 128;

  // ---- bias of a tile: wave w moves the tile's columns [32 w, 32 w + 32) into LDS slot
  // (tile index & 1) with one LDS-DMA load (columns past o read a valid column; the
  // stores of those columns are dropped) ----
  lds_char* const bias_lds = smem + 2 * kXlStageBytes + 8 * kX8StripBytes;
  auto lane_now = []() {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
  };
  const char* const bias_base = p.bias ? static_cast<const char*>(p.bias) : static_cast<const char*>(p.c);
  auto load_bias = [&](const Tile& t, int slot) {
    constexpr int EPC = 16 / static_cast<int>(sizeof(TB));       // bias elements per 16-byte chunk
    constexpr int LANES = 32 / EPC;                               // lanes that move the wave's 32 columns
    const int ln = lane_now();
    const int col = t.o0 + 32 * wave + EPC * (ln < LANES ? ln : 0);
    const int cl = col < p.o ? col : p.o - EPC;
    const int64_t eoff = p.bias ? static_cast<int64_t>(t.mdl) * p.b_sn + cl : 0;
    if (ln < LANES)
      __builtin_amdgcn_global_load_lds(bias_base + eoff * static_cast<int64_t>(sizeof(TB)),
                                       (lds_ptr_t)(bias_lds + slot * kXlBiasSlot + 32 * wave * sizeof(TB)), 16, 0, 0);
  };

  // acc[i][j]: W rows ow + 16 i, A rows mw + 16 j; lane (g = lane >> 4, fr) holds C
  // columns ow + 16 i + 4 g + e of row mw + 16 j + fr
  f32x4 acc[8][4];

  // ---- epilogue of tile t: acc (+ bias, ReLU) -> C, one 16-row x 64-column half strip at
  // a time through LDS, then 16-byte row chunks: lane -> row 8 q + (lane >> 3), 8 columns
  // from 8 (lane & 7) ----
  lds_char* strip = smem + 2 * kXlStageBytes + wave * kX8StripBytes;
  auto epilogue = [&](const Tile& t, int ti_parity) {
    const __amdgpu_buffer_rsrc_t crs =
        xl_rsrc(static_cast<TA*>(p.c) + static_cast<int64_t>(t.mdl) * p.c_sn, p.c_bytes);
    const int ln = lane_now();
    const int fr = ln & 15, g4 = ln >> 4;
    if (KS == 1) {
      vm_lgkm_wait<0>();
      bare_barrier();
    }
    const int rr = ln >> 3, cc = ln & 7;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      // bias of the lane's columns ow + 64 hh + 16 i' + 4 g4 + e
      float bv[4][4];
      const lds_char* bl = bias_lds + (ti_parity & 1) * kXlBiasSlot + (ow + 64 * hh + 4 * g4) * sizeof(TB);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (sizeof(TB) == 4) {
          const f32x4 b4 = *(const __attribute__((address_space(3))) f32x4*)(bl + 16 * i * 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) bv[i][e] = p.bias ? b4[e] : 0.f;
        } else {
          typedef TB tb4 __attribute__((ext_vector_type(4)));
          typedef __attribute__((address_space(3))) tb4 lds_tb4;
          const auto b4 = *(const lds_tb4*)(bl + 16 * i * 2);
#pragma unroll
          for (int e = 0; e < 4; ++e) bv[i][e] = p.bias ? to_f32(b4[e]) : 0.f;
        }
      }
      const int col = t.o0 + ow + 64 * hh + cc * 8;
      const bool col_ok = col < p.o;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          bf16x4 o4;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float v = acc[4 * hh + i][j][e] + bv[i][e];
            if (RELU) v = relu_f(v);
            o4[e] = __builtin_bit_cast(bf16, from_f32<TA>(v));   // the strip holds raw 16-bit values
          }
          *(lds_bf16x4*)(strip + fr * kX8StripPitch + (16 * i + 4 * g4) * 2) = o4;
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);          // lgkmcnt(0): half strip written
        __builtin_amdgcn_wave_barrier();
        // the strip's 16 rows share one row decomposition (rows_inner % 16 == 0)
        const int row0 = t.m0 + mw + 16 * j;
        const uint32_t outer = fdiv(static_cast<uint32_t>(row0), p.c_ri);
        const uint32_t inner = row0 - outer * p.c_ri.d;
        const bool strip_ok = row0 < p.m && col_ok;
        const uint32_t cbase =
            (outer * static_cast<uint32_t>(p.c_so) + inner * static_cast<uint32_t>(p.c_si) + col) * 2u;
        i32x4 raw[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) raw[q] = *(const lds_i32x4*)(strip + (8 * q + rr) * kX8StripPitch + cc * 16);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const int lr = 8 * q + rr;
          // non-temporal at device scope (nt | sc1): the output streams past the L2s, which keep
          // the operand tiles (vocabulary-shape launch 1099-1101 against 1104-1111 µs with nt
          // alone, and the kernels after it in a step find more of their operands cached)
          __builtin_amdgcn_raw_buffer_store_b128(
              raw[q], crs, strip_ok ? cbase + static_cast<uint32_t>(lr * p.c_si) * 2u : kXlOob, 0, 18);
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);          // strip reads done before it is rewritten
        __builtin_amdgcn_wave_barrier();
      }
    }
  };

  // ---- main loop, software-pipelined within each wave.  A stage is 16 groups of 4
  // MFMAs: group g = 8 h + i multiplies W fragment i of K half h with the 4 A fragments
  // of that half.  W fragments stream through a ring of 4 registers, read 4 groups ahead
  // (after group g's MFMAs, fragment g + 4 into g's ring slot); the A fragments of half 1
  // are read during half 0 and those of the next stage's half 0 after the stage's barrier,
  // which sits after group 13: by then every fragment of the stage has been read, and the
  // 8 MFMAs of groups 14 and 15 are issued beside the next stage's first reads and the
  // DMA of stage s + 2.  A wave therefore rarely waits for its own LDS reads. ----
  bf16x8 wr[4], a0[4], a1[4];
  auto rd_w = [&](int stage, int g) {
    const lds_char* st = smem + (stage & 1) * kXlStageBytes + ((g >> 3) ? fp1 : fp0);
    wr[g & 3] = *(const lds_bf16x8*)(st + wfo + (g & 7) * 2048);
  };
  auto rd_a = [&](int stage, int h, bf16x8 (&a)[4]) {
    const lds_char* st = smem + (stage & 1) * kXlStageBytes + (h ? fp1 : fp0);
#pragma unroll
    for (int j = 0; j < 4; ++j) a[j] = *(const lds_bf16x8*)(st + afo + j * 2048);
  };
  auto group = [&](int g, bf16x8 (&a)[4], bool zero) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[g & 7][j] = mma16<TA>(wr[g & 3], a[j], zero ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[g & 7][j]);
  };
  // prologue: stage 0 landed, stage 1 in flight, stage 0's first reads issued
  issue(0);
  load_bias(tile_of(0), 0);
  vm_lgkm_wait<0>();
  bare_barrier();
  issue(1);
#pragma unroll
  for (int g = 0; g < 4; ++g) rd_w(0, g);
  rd_a(0, 0, a0);

  auto stage = [&](int s, bool first, bool after_epi) {
    Dma d;
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      if (g < 14) {
        group(g, g < 8 ? a0 : a1, first && g < 8);
      } else {
        // groups 14 and 15: one of stage s + 2's 8 LDS-DMA loads after each MFMA (issued
        // back to back they stall the wave while the address unit drains them)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[g & 7][j] = mma16<TA>(wr[g & 3], a1[j], acc[g & 7][j]);
          __builtin_amdgcn_sched_barrier(0);
          dma_block(d, 4 * (g - 14) + j);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      if (g == 1) rd_a(s, 1, a1);                     // a1 last fed group 15 of stage s - 1
      if (g + 4 < 16) rd_w(s, g + 4);
      if (g == 13) {
        // every read of stage s issued (the last after group 11); stage s + 1 landed:
        // then slot s & 1 can take stage s + 2 and stage s + 1 can be read
        if (after_epi) vm_lgkm_wait<E>();
        else vm_lgkm_wait<0>();
        bare_barrier();
        rd_a(s + 1, 0, a0);                           // a0 last fed group 7
        rd_w(s + 1, 0);
        rd_w(s + 1, 1);
        d = dma_of(s + 2);
      }
      if (g == 14) rd_w(s + 1, 2);
      if (g == 15) rd_w(s + 1, 3);
    }
  };

  for (int ti = 0; ti < my_tiles; ++ti) {
    stage(ti * KS, true, ti > 0);
    for (int ks = 1; ks < KS; ++ks) stage(ti * KS + ks, false, false);
    epilogue(tile_of(ti), ti);
    load_bias(tile_of(ti + 1 < my_tiles ? ti + 1 : ti), (ti + 1) & 1);
  }
  vm_lgkm_wait<0>();                               // no LDS-DMA load outlives the workgroup
}

// Elements from one model's base to the end of the last of its m rows (of `width`
// columns) addressed as (m / ri) * so + (m % ri) * si.
inline int64_t xl_span(const GemmParams& p, int64_t so, int64_t si, int64_t ri, int64_t width) {
  const int64_t outer = (p.m - 1) / ri;
  const int64_t inner = p.m - 1 < ri ? p.m - 1 : ri - 1;
  return outer * so + inner * si + width;
}


template <typename TA, typename TB>
int32_t launch_xl(GemmParams p, hipStream_t st) {
  p.tiles_m = static_cast<int>(cdiv(p.m, kXlB));
  p.tiles_o = static_cast<int>(cdiv(p.o, kXlB));
  const int64_t tiles = static_cast<int64_t>(p.n) * p.tiles_m * p.tiles_o;
  if (tiles >= 0x7fffffffll) return set_error(WC_ERR_LIMIT, "wc_grouped_gemm: too many tiles");
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
      return set_error(WC_ERR_ARG, "wc_grouped_gemm: cannot query the CU count");
    cus = v;
  }
  const int grid = static_cast<int>(tiles < cus ? tiles : cus);
  // bf16 C / R (the only XL output type); xl_shape_ok has bounded both below 2^31
  p.c_bytes = static_cast<int32_t>(xl_span(p, p.c_so, p.c_si, p.c_ri.d, p.o) * 2);
  p.r_bytes = p.r ? static_cast<int32_t>(xl_span(p, p.r_so, p.r_si, p.c_ri.d, p.o) * 2) : p.c_bytes;
  p.fd_ks = make_fastdiv(static_cast<uint32_t>(p.k / kXlBK));
  p.fd_tpm = make_fastdiv(static_cast<uint32_t>(p.tiles_m * p.tiles_o));
  p.fd_tm = make_fastdiv(static_cast<uint32_t>(p.tiles_m));
  const bool relu = p.act == WC_ACT_RELU;
  if (!p.r) {
    auto kern8 = relu ? gemm_xl8_kernel<TA, TB, true> : gemm_xl8_kernel<TA, TB, false>;
    kern8<<<dim3(grid), dim3(kX8Threads), 0, st>>>(p, static_cast<int>(tiles));
    return check_launch("wc_grouped_gemm");
  }
  auto kern = relu ? gemm_xlp_kernel<TA, TB, true, true> : gemm_xlp_kernel<TA, TB, true, false>;
  kern<<<dim3(grid), dim3(kXlThreads), 0, st>>>(p, static_cast<int>(tiles));
  return check_launch("wc_grouped_gemm");
}

template <typename TA, typename TC, typename TB, int WM, int WN, int FM, int FN>
int32_t launch_big(GemmParams p, hipStream_t st) {
  using C = BigCfg<WM, WN, FM, FN>;
  p.tiles_m = static_cast<int>(cdiv(p.m, C::BM));
  p.tiles_o = static_cast<int>(cdiv(p.o, C::BN));
  const int64_t nblk = static_cast<int64_t>(p.n) * p.tiles_m * p.tiles_o;
  if (nblk >= 0x7fffffffll) return set_error(WC_ERR_LIMIT, "wc_grouped_gemm: too many tiles");
  p.remap = (nblk % 8 == 0) ? 1 : 0;
  auto kern = gemm_big_kernel<TA, TC, TB, WM, WN, FM, FN>;
  if (C::LDS > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(C::LDS));
    if (e != hipSuccess)
      return set_error(static_cast<int32_t>(e), "wc_grouped_gemm: LDS of %zu bytes refused: %s", C::LDS,
                       hipGetErrorString(e));
  }
  kern<<<dim3(static_cast<uint32_t>(nblk)), dim3(C::NT), C::LDS, st>>>(p);
  return check_launch("wc_grouped_gemm");
}

template <typename TA, typename TC, typename TB, int TM, int TN, int WM, int WN>
int32_t launch_cfg(GemmParams p, bool vec, hipStream_t st) {
  constexpr int BM = WM * TM, BN = WN * TN;
  p.tiles_m = static_cast<int>(cdiv(p.m, BM));
  p.tiles_o = static_cast<int>(cdiv(p.o, BN));
  const int64_t nblk = static_cast<int64_t>(p.n) * p.tiles_m * p.tiles_o;
  if (nblk >= 0x7fffffffll) return set_error(WC_ERR_LIMIT, "wc_grouped_gemm: too many tiles");
  p.remap = (nblk % 8 == 0) ? 1 : 0;
  const dim3 grid(static_cast<uint32_t>(nblk)), block(WM * WN * 64);
  if (vec)
    gemm_kernel<TA, TC, TB, TM, TN, WM, WN, true><<<grid, block, 0, st>>>(p);
  else
    gemm_kernel<TA, TC, TB, TM, TN, WM, WN, false><<<grid, block, 0, st>>>(p);
  return check_launch("wc_grouped_gemm");
}

// Shapes the persistent XL kernel takes: K a multiple of 64 (an even number of
// 32-wide stages), M, O and both rows_inner multiples of 16 (a 16-row block
// never straddles an outer row group), 16-byte aligned output / residual rows
// and per-model byte offsets below 2^31 (32-bit DMA and buffer offsets).
template <typename TC>
bool xl_shape_ok(const GemmParams& p) {
  const int64_t es = sizeof(TC);
  if (p.k % 64 != 0 || p.m % 16 != 0 || p.o % 16 != 0 || p.a_ri.d % 16 != 0 || p.c_ri.d % 16 != 0) return false;
  if (p.a_so < 0 || p.a_si < 0 || p.c_so < 0 || p.c_si < 0 || p.r_so < 0 || p.r_si < 0) return false;
  const bool c_ok = common_vec_bytes({reinterpret_cast<uintptr_t>(p.c), ubytes(p.c_sn, es),
                                      ubytes(p.c_so, es), ubytes(p.c_si, es)}) >= 16;
  const bool r_ok = !p.r || common_vec_bytes({reinterpret_cast<uintptr_t>(p.r), ubytes(p.r_sn, es),
                                              ubytes(p.r_so, es),
                                              ubytes(p.r_si, es)}) >= 16;
  if (!c_ok || !r_ok) return false;
  const int64_t lim = 0x7fffffffll;
  const int64_t a_end = xl_span(p, p.a_so, p.a_si, p.a_ri.d, p.k) * 2;
  const int64_t w_end = static_cast<int64_t>(p.o) * p.k * 2;
  const int64_t c_end = xl_span(p, p.c_so, p.c_si, p.c_ri.d, p.o) * es;
  const int64_t r_end = p.r ? xl_span(p, p.r_so, p.r_si, p.c_ri.d, p.o) * es : 0;
  return a_end < lim && w_end < lim && c_end < lim && r_end < lim;
}

template <typename TA, typename TC, typename TB>
int32_t launch_gemm_t(const GemmParams& p, bool vec, hipStream_t st) {
  if constexpr (sizeof(TA) == 2) {
    const int64_t tiles256 = static_cast<int64_t>(p.n) * cdiv(p.m, 256) * cdiv(p.o, 256);
    if constexpr (sizeof(TC) == 2)
      if (vec && tiles256 >= 256 && xl_shape_ok<TC>(p)) return launch_xl<TA, TB>(p, st);
    if (vec && tiles256 >= 256) return launch_big<TA, TC, TB, 2, 4, 8, 4>(p, st);
  }
  const int64_t tiles128 = static_cast<int64_t>(p.n) * cdiv(p.m, 128) * cdiv(p.o, 128);
  if (tiles128 >= 512) return launch_cfg<TA, TC, TB, 64, 64, 2, 2>(p, vec, st);
  const int64_t tiles64 = static_cast<int64_t>(p.n) * cdiv(p.m, 64) * cdiv(p.o, 64);
  if (tiles64 >= 1024) return launch_cfg<TA, TC, TB, 32, 32, 2, 2>(p, vec, st);
  // small problems are latency-bound: 16 x 16 wave tiles give each wave the
  // fewest dependent MFMAs and the most workgroups in flight
  return launch_cfg<TA, TC, TB, 16, 16, 2, 2>(p, vec, st);
}

}  // namespace

// Internal entry shared by other kernel families (e.g. the recurrent input
// projection).  Dtypes: A/W in {f32, bf16}; C f32 or == A; bias f32 or == A.
int32_t grouped_gemm(const GemmParams& p0, int32_t dtype, int32_t out_dtype, int32_t bias_dtype,
                     hipStream_t st) {
  GemmParams p = p0;
  const int es = dtype_size(dtype);
  const bool vec = common_vec_bytes({reinterpret_cast<uintptr_t>(p.a), reinterpret_cast<uintptr_t>(p.w),
                                     ubytes(p.k, es), ubytes(p.a_sn, es),
                                     ubytes(p.a_so, es), ubytes(p.a_si, es),
                                     ubytes(p.w_sn, es)}) >= 16;
  if (dtype == WC_F32) {
    if (out_dtype != WC_F32 || (p.bias && bias_dtype != WC_F32))
      return set_error(WC_ERR_DTYPE, "wc_grouped_gemm: f32 inputs need f32 output and bias");
    return launch_gemm_t<float, float, float>(p, vec, st);
  }
  if (dtype == WC_BF16) {
    const bool bias_f32 = p.bias && bias_dtype == WC_F32;
    if (p.bias && bias_dtype != WC_F32 && bias_dtype != WC_BF16)
      return set_error(WC_ERR_DTYPE, "wc_grouped_gemm: bias dtype %s", dtype_name(bias_dtype));
    if (out_dtype == WC_BF16)
      return bias_f32 ? launch_gemm_t<bf16, bf16, float>(p, vec, st)
                      : launch_gemm_t<bf16, bf16, bf16>(p, vec, st);
    if (out_dtype == WC_F32)
      return bias_f32 ? launch_gemm_t<bf16, float, float>(p, vec, st)
                      : launch_gemm_t<bf16, float, bf16>(p, vec, st);
    return set_error(WC_ERR_DTYPE, "wc_grouped_gemm: output dtype %s", dtype_name(out_dtype));
  }
  if (dtype == WC_F16) {
    const bool bias_f32 = p.bias && bias_dtype == WC_F32;
    if (p.bias && bias_dtype != WC_F32 && bias_dtype != WC_F16)
      return set_error(WC_ERR_DTYPE, "wc_grouped_gemm: bias dtype %s", dtype_name(bias_dtype));
    if (out_dtype == WC_F16)
      return bias_f32 ? launch_gemm_t<f16, f16, float>(p, vec, st) : launch_gemm_t<f16, f16, f16>(p, vec, st);
    if (out_dtype == WC_F32)
      return bias_f32 ? launch_gemm_t<f16, float, float>(p, vec, st) : launch_gemm_t<f16, float, f16>(p, vec, st);
    return set_error(WC_ERR_DTYPE, "wc_grouped_gemm: output dtype %s", dtype_name(out_dtype));
  }
  return set_error(WC_ERR_DTYPE, "wc_grouped_gemm: unsupported dtype %s", dtype_name(dtype));
}

}  // namespace wc

using namespace wc;

extern "C" int32_t wc_grouped_gemm(const wc_gemm_args* g, void* stream) {
  clear_error();
  WC_REQUIRE(g != nullptr, WC_ERR_NULL, "wc_grouped_gemm: null args");
  WC_REQUIRE(g->n >= 0 && g->m >= 0 && g->o >= 0 && g->k >= 0, WC_ERR_SHAPE,
             "wc_grouped_gemm: negative size");
  if (g->n == 0 || g->m == 0 || g->o == 0) return WC_OK;
  WC_REQUIRE(g->a && g->w && g->c, WC_ERR_NULL, "wc_grouped_gemm: null pointer");
  WC_REQUIRE(g->act == WC_ACT_NONE || g->act == WC_ACT_RELU, WC_ERR_ARG, "wc_grouped_gemm: bad act");
  WC_REQUIRE(g->m < 0x7fffffffll && g->o < 0x7fffffffll && g->k < 0x7fffffffll && g->n < 0x7fffffffll,
             WC_ERR_LIMIT, "wc_grouped_gemm: sizes too large");
  WC_REQUIRE(g->a_rows_inner > 0 && g->c_rows_inner > 0, WC_ERR_ARG,
             "wc_grouped_gemm: rows_inner must be positive");
  WC_REQUIRE(g->a_rows_inner < 0x7fffffffll && g->c_rows_inner < 0x7fffffffll, WC_ERR_LIMIT,
             "wc_grouped_gemm: rows_inner too large");
  WC_REQUIRE(g->residual == nullptr || g->out_dtype == g->dtype || g->out_dtype == WC_F32,
             WC_ERR_DTYPE, "wc_grouped_gemm: residual dtype");
  GemmParams p;
  p.n = (int)g->n;
  p.m = (int)g->m;
  p.o = (int)g->o;
  p.k = (int)g->k;
  p.act = g->act;
  p.a = g->a;
  p.a_sn = g->a_stride_n;
  p.a_so = g->a_stride_outer;
  p.a_si = g->a_stride_inner;
  p.a_ri = make_fastdiv(static_cast<uint32_t>(g->a_rows_inner));
  p.w = g->w;
  p.w_sn = g->w_stride_n;
  p.bias = g->bias;
  p.b_sn = g->bias_stride_n;
  p.r = g->residual;
  p.r_sn = g->r_stride_n;
  p.r_so = g->r_stride_outer;
  p.r_si = g->r_stride_inner;
  p.c = g->c;
  p.c_sn = g->c_stride_n;
  p.c_so = g->c_stride_outer;
  p.c_si = g->c_stride_inner;
  p.c_ri = make_fastdiv(static_cast<uint32_t>(g->c_rows_inner));
  return grouped_gemm(p, g->dtype, g->out_dtype, g->bias_dtype, as_stream(stream));
}
