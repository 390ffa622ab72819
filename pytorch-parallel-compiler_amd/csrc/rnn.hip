// Persistent recurrent kernels (GRU / LSTM forward, one layer, unidirectional).
//
// Two launches.  (1) The input projection gates_x = x W_ih^T + b_ih for all
// steps at once, as a grouped MFMA GEMM into an fp32 workspace [N, B*T, G]
// (the reference computes the same einsum before its time loop).  (2) The
// recurrence: one workgroup owns one (model, batch row) pair for all T steps;
// batch rows never interact in a recurrence, so no cross-workgroup
// synchronisation is needed.  Every lane holds a K-slice of one gate row of
// W_hh in registers for the whole sequence (loaded once).
//
// The step loop issues no vector-memory instruction at all: gates_x for a
// chunk of XT steps is staged into LDS with coalesced loads before the chunk,
// and the chunk's hidden states are collected in LDS and written out with
// coalesced stores after it.  (Global loads and stores in flight together
// inside the loop make the compiler wait for all outstanding memory at every
// iteration, exposing the full memory latency once per step.)
//
// Lane layout: lanes form groups of LG = 8 or 16 adjacent lanes (a DPP
// half-row or row).  Group g owns UPG hidden units u = g*UPG + k and therefore
// the GATES*UPG gate rows q*H + u of W_hh; lane j of the group holds columns
// [j*KL, (j+1)*KL) of those rows in registers (loaded once, 16-byte vector
// loads).  Per step a lane reads only its KL hidden values from LDS (padded,
// bank-conflict-free layout), forms GATES*UPG partial dot products and folds
// them across the group with log2(LG) DPP butterfly adds (no LDS traffic).
// Lane k < UPG of the group then applies the cell update of unit g*UPG + k and
// writes h into LDS; one barrier per step.
#include <type_traits>

#include "wc_gemm.h"
#include "wc_rnn.h"

namespace wc {
namespace {

constexpr int kRnnLdsBudget = 144 * 1024;   // of gfx950's 160 KB per workgroup

struct RnnParams {
  int n, batch, steps, in, hid;
  int lg;             // lanes per group (8 or 16)
  int kl;             // hidden columns per lane (multiple of 4)
  int upg;            // hidden units per group
  int wvec;           // W_hh rows can be read with 16-byte vector loads
  int xt;             // steps per LDS chunk of gates_x / outputs
  int remap;          // XCD-aware workgroup order
  const float* gx;    // [N, B, T, G] fp32 input projection incl. b_ih
  const void* w_hh;
  const void* b_hh;
  const void* h0;
  const void* c0;
  void* out;
  void* hn;
  void* cn;
};

// DPP lane permutations inside a 16-lane row (register-to-register, no LDS)
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF,
                                                               0xF, true));
}

// sum over groups of LG adjacent lanes (2, 4: part of a quad; 8: half-row;
// 16: row), delivered to every lane of the group
template <int LG>
__device__ __forceinline__ float group_sum_dpp(float v) {
  static_assert(LG == 2 || LG == 4 || LG == 8 || LG == 16, "group size");
  v += dpp<0xB1>(v);                  // quad_perm [1,0,3,2]
  if (LG >= 4) v += dpp<0x4E>(v);     // quad_perm [2,3,0,1]
  if (LG >= 8) v += dpp<0x141>(v);    // row_half_mirror: lane i <- 7 - i within each 8 lanes
  if (LG == 16) v += dpp<0x140>(v);   // row_mirror: lane i <- 15 - i
  return v;
}

// KL consecutive elements of a W_hh row as floats (16-byte loads when allowed)
template <typename T, int KL>
__device__ __forceinline__ void load_cols(const T* row, int col0, int h, bool vec, float* dst) {
  constexpr int VE = 16 / sizeof(T);
  if (vec && col0 + KL <= h) {
#pragma unroll
    for (int i = 0; i < KL; i += VE) {
      if constexpr (sizeof(T) == 4) {
        const float4 v = *reinterpret_cast<const float4*>(row + col0 + i);
        dst[i] = v.x;
        dst[i + 1] = v.y;
        dst[i + 2] = v.z;
        dst[i + 3] = v.w;
      } else {
        typedef T t8 __attribute__((ext_vector_type(8)));
        const t8 v = *reinterpret_cast<const t8*>(row + col0 + i);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (i + e < KL) dst[i + e] = static_cast<float>(v[e]);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < KL; ++i) dst[i] = (col0 + i < h) ? to_f32(row[col0 + i]) : 0.f;
  }
}

template <typename T>
__device__ __forceinline__ float ldf(const void* p, int64_t i) {
  return to_f32(static_cast<const T*>(p)[i]);
}

// LDS-only barrier: waits for this wave's LDS traffic, not for its global
// loads, so the gates_x prefetches stay in flight across steps.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Lanes holding more than 64 weight registers run at most 8 waves per
// workgroup (two per SIMD), which doubles the VGPRs each may use.
constexpr int rnn_bound(int gates, int upg, int kl) { return gates * upg * kl > 64 ? 512 : 1024; }

template <typename T, int CELL, int LG, int UPG, int KL>
__global__ __launch_bounds__(rnn_bound(CELL == WC_CELL_GRU ? 3 : 4, UPG, KL)) void rnn_seq_kernel(RnnParams p) {
  constexpr int GATES = (CELL == WC_CELL_GRU) ? 3 : 4;
  constexpr int KLP = KL + 4;                        // padded LDS pitch per lane slice
  constexpr int HP = LG * KLP;                       // padded h buffer length
  const int H = p.hid;
  const int G = GATES * H;
  extern __shared__ float4 smem4[];
  float* sh_h = reinterpret_cast<float*>(smem4);    // [2][HP]
  float* sgx = sh_h + 2 * HP;                        // [xt][G]
  float* sout = sgx + static_cast<int64_t>(p.xt) * G;  // [xt][H]

  // workgroup -> (model, batch row); with remap, consecutive ids (the batch
  // rows of one model, which read the same weights) share an XCD's L2.
  const int nwg = p.n * p.batch;
  int id = blockIdx.x;
  if (p.remap) id = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);
  const int mdl = id / p.batch;
  const int bb = id - mdl * p.batch;

  const int tid = threadIdx.x;
  const int nthreads = blockDim.x;
  const int j = tid & (LG - 1);           // lane in the group
  const int grp = tid / LG;               // group
  const int u0 = grp * UPG;               // first unit of the group

  // ---- registers: W_hh[q*H + u0 + k][j*KL .. +KL] and b_hh ----
  float w[UPG][GATES][KL];
  float bhh[UPG][GATES];
  {
    const T* wb = static_cast<const T*>(p.w_hh) + static_cast<int64_t>(mdl) * G * H;
#pragma unroll
    for (int k = 0; k < UPG; ++k)
#pragma unroll
      for (int q = 0; q < GATES; ++q) {
        const int u = u0 + k;
        if (u < H) {
          load_cols<T, KL>(wb + static_cast<int64_t>(q * H + u) * H, j * KL, H, p.wvec != 0, w[k][q]);
        } else {
#pragma unroll
          for (int i = 0; i < KL; ++i) w[k][q][i] = 0.f;
        }
        bhh[k][q] = (u < H && p.b_hh) ? ldf<T>(p.b_hh, static_cast<int64_t>(mdl) * G + q * H + u) : 0.f;
      }
  }

  // ---- LDS init: h0 in the padded layout, zeros elsewhere ----
  const int64_t st_off = (static_cast<int64_t>(mdl) * p.batch + bb) * H;  // [n, b, H] offset
  for (int e = tid; e < 2 * HP; e += nthreads) {
    const int pos = e < HP ? e : e - HP;
    const int sl = pos / KLP, off = pos - sl * KLP;
    const int col = sl * KL + off;
    float v = 0.f;
    if (e < HP && off < KL && col < H && p.h0) v = ldf<T>(p.h0, st_off + col);
    sh_h[e] = v;
  }
  const int my_u = u0 + j;                     // unit updated by this lane (j < UPG)
  const bool leader = (j < UPG) && (my_u < H);
  const int my_pos = (my_u / KL) * KLP + (my_u % KL);
  float h_reg = 0.f, c_reg = 0.f;
  if (leader) {
    h_reg = p.h0 ? ldf<T>(p.h0, st_off + my_u) : 0.f;
    if (CELL == WC_CELL_LSTM) c_reg = p.c0 ? ldf<T>(p.c0, st_off + my_u) : 0.f;
  }
  T* outb = static_cast<T*>(p.out) + (static_cast<int64_t>(mdl) * p.batch + bb) *
                                          static_cast<int64_t>(p.steps) * H;
  const float* gxb = p.gx + (static_cast<int64_t>(mdl) * p.batch + bb) * static_cast<int64_t>(p.steps) * G;

  int prev_t0 = 0, prev_nt = 0;
  for (int t0 = 0; t0 < p.steps; t0 += p.xt) {
    const int nt = (p.steps - t0 < p.xt) ? (p.steps - t0) : p.xt;
    // flush the previous chunk's hidden states (contiguous rows of out)
    for (int e = tid; e < prev_nt * H; e += nthreads)
      outb[static_cast<int64_t>(prev_t0) * H + e] = from_f32<T>(sout[e]);
    // stage this chunk's gates_x (contiguous in the workspace)
    const float4* src4 = reinterpret_cast<const float4*>(gxb + static_cast<int64_t>(t0) * G);
    float4* dst4 = reinterpret_cast<float4*>(sgx);
    for (int e = tid; e < (nt * G) >> 2; e += nthreads) dst4[e] = src4[e];
    for (int e = ((nt * G) & ~3) + tid; e < nt * G; e += nthreads)
      sgx[e] = gxb[static_cast<int64_t>(t0) * G + e];
    __syncthreads();

    for (int tt = 0; tt < nt; ++tt) {
      const int cur = (t0 + tt) & 1;
      // this step's gates_x of the lane's unit, read before the dot products so
      // its LDS latency is off the critical path (non-leaders read a valid slot)
      float gxv[GATES];
      {
        const float* gxt = sgx + tt * G + (leader ? my_u : 0);
#pragma unroll
        for (int q = 0; q < GATES; ++q) gxv[q] = gxt[q * H];
      }
      float hv[KL];
      const float* hs = sh_h + cur * HP + j * KLP;
#pragma unroll
      for (int i = 0; i < KL; i += 4) {
        const float4 a = *reinterpret_cast<const float4*>(hs + i);
        hv[i] = a.x;
        hv[i + 1] = a.y;
        hv[i + 2] = a.z;
        hv[i + 3] = a.w;
      }
      // gates_h = h W_hh^T + b_hh for the group's rows, summed over the group
      float gh[UPG][GATES];
#pragma unroll
      for (int k = 0; k < UPG; ++k)
#pragma unroll
        for (int q = 0; q < GATES; ++q) {
          float acc = 0.f;
#pragma unroll
          for (int i = 0; i < KL; ++i) acc += w[k][q][i] * hv[i];
          gh[k][q] = group_sum_dpp<LG>(acc) + bhh[k][q];
        }
      if (leader) {
        // this lane's unit: pick its gates from the group sums (j == k)
        float g_h[GATES];
#pragma unroll
        for (int q = 0; q < GATES; ++q) {
          g_h[q] = gh[0][q];
#pragma unroll
          for (int k = 1; k < UPG; ++k)
            if (j == k) g_h[q] = gh[k][q];
        }
        float hnew;                                // gates_x = x W_ih^T + b_ih in gxv
        if (CELL == WC_CELL_GRU) {
          const float rg = sigmoid_f(gxv[0] + g_h[0]);
          const float zg = sigmoid_f(gxv[1] + g_h[1]);
          const float nn = tanh_f(gxv[2] + rg * g_h[2]);
          hnew = (1.0f - zg) * nn + zg * h_reg;
        } else {
          const float ig = sigmoid_f(gxv[0] + g_h[0]);
          const float fg = sigmoid_f(gxv[1] + g_h[1]);
          const float gg = tanh_f(gxv[2] + g_h[2]);
          const float og = sigmoid_f(gxv[3] + g_h[3]);
          c_reg = fg * c_reg + ig * gg;
          hnew = og * tanh_f(c_reg);
        }
        h_reg = hnew;
        sh_h[(cur ^ 1) * HP + my_pos] = hnew;
        sout[tt * H + my_u] = hnew;
      }
      lds_barrier();
    }
    prev_t0 = t0;
    prev_nt = nt;
  }
  for (int e = tid; e < prev_nt * H; e += nthreads)
    outb[static_cast<int64_t>(prev_t0) * H + e] = from_f32<T>(sout[e]);
  if (leader) {
    if (p.hn) static_cast<T*>(p.hn)[st_off + my_u] = from_f32<T>(h_reg);
    if (CELL == WC_CELL_LSTM && p.cn) static_cast<T*>(p.cn)[st_off + my_u] = from_f32<T>(c_reg);
  }
}

template <typename K>
int32_t launch_lds(K kernel, const RnnParams& p, dim3 grid, dim3 block, size_t lds, hipStream_t st) {
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess)
      return set_error(static_cast<int32_t>(e), "wc_rnn_recurrence: LDS of %zu bytes refused: %s", lds,
                       hipGetErrorString(e));
  }
  kernel<<<grid, block, lds, st>>>(p);
  return check_launch("wc_rnn_recurrence");
}

template <typename T, int CELL, int LG, int UPG, int KL>
int32_t launch_one(const RnnParams& p, dim3 grid, dim3 block, size_t lds, hipStream_t st) {
  return launch_lds(rnn_seq_kernel<T, CELL, LG, UPG, KL>, p, grid, block, lds, st);
}

// The (lanes per group, units per group, columns per lane) shapes rnn_plan may pick.
template <typename T, int CELL>
int32_t launch_rec(const RnnParams& p, dim3 grid, dim3 block, size_t lds, hipStream_t st) {
#define WC_RNN_SHAPE(LG, UPG, KL)                      \
  if (p.lg == LG && p.upg == UPG && p.kl == KL) \
    return launch_one<T, CELL, LG, UPG, KL>(p, grid, block, lds, st);
  WC_RNN_SHAPE(16, 1, 4) WC_RNN_SHAPE(16, 2, 4) WC_RNN_SHAPE(16, 4, 4)
  WC_RNN_SHAPE(16, 1, 8) WC_RNN_SHAPE(16, 2, 8) WC_RNN_SHAPE(16, 4, 8)
  WC_RNN_SHAPE(16, 1, 16) WC_RNN_SHAPE(16, 2, 16) WC_RNN_SHAPE(16, 4, 16)
  WC_RNN_SHAPE(8, 1, 4) WC_RNN_SHAPE(8, 2, 4) WC_RNN_SHAPE(8, 4, 4)
  WC_RNN_SHAPE(8, 1, 8) WC_RNN_SHAPE(8, 2, 8) WC_RNN_SHAPE(8, 4, 8)
  WC_RNN_SHAPE(8, 1, 16) WC_RNN_SHAPE(8, 2, 16) WC_RNN_SHAPE(8, 4, 16)
  WC_RNN_SHAPE(4, 1, 8) WC_RNN_SHAPE(4, 2, 8)
  WC_RNN_SHAPE(4, 1, 16) WC_RNN_SHAPE(4, 2, 16)
  WC_RNN_SHAPE(4, 1, 32)
  WC_RNN_SHAPE(2, 1, 32)
#undef WC_RNN_SHAPE
  return set_error(WC_ERR_LIMIT, "wc_rnn_recurrence: no kernel for %d lanes x %d units x %d columns", p.lg,
                   p.upg, p.kl);
}

inline int round_up(int v, int m) { return (v + m - 1) / m * m; }

// ---------------------------------------------------------------------------
// Streamed recurrence for hidden sizes whose W_hh does not fit one workgroup:
// one launch per time step.  Workgroup = (model, block of UB units); it forms
// the gate pre-activations of its units for all batch rows as an MFMA GEMM
//   G[b][r] = sum_k h_{t-1}[b][k] W_hh[row(r)][k],   row(r) = (r / UB)*H + u0 + r % UB
// with A = h_{t-1} (batch rows, read from the previous step's output) and
// B = the W_hh rows (K-contiguous, streamed from L2 / MALL), stages G in LDS,
// then applies the cell update for its (batch row, unit) pairs.  The cell
// state is carried in an fp32 workspace.
// ---------------------------------------------------------------------------
struct StepParams {
  int n, batch, steps, hid, t, ublocks;
  const void* hprev;          // h_{t-1}: [n][batch] rows of `hid` elements (null: zeros)
  int64_t hp_sn, hp_sb;
  const float* gx;            // [n, batch, steps, G] fp32 (incl. b_ih)
  const void* w_hh;           // [n, G, hid]
  const void* b_hh;           // [n, G] or null
  float* cst;                 // [n, batch, hid] fp32 cell state (LSTM)
  const void* c0;             // initial cell state or null (read at t == 0)
  void* out;                  // [n, batch, steps, hid]
  void* hn;
  void* cn;
};

constexpr int kStepThreads = 256;

template <typename T, int CELL>
struct StepCfg {
  static constexpr int GATES = CELL == WC_CELL_GRU ? 3 : 4;
  static constexpr int NTW = CELL == WC_CELL_GRU ? 3 : 2;   // 16-row tiles per wave
  static constexpr int R = 4 * 16 * NTW;                     // gate rows per workgroup
  static constexpr int UB = R / GATES;                       // units per workgroup (64 / 32)
};

template <typename T, int CELL>
__global__ __launch_bounds__(kStepThreads, CELL == WC_CELL_GRU ? 2 : 4) void rnn_step_kernel(StepParams p) {
  using C = StepCfg<T, CELL>;
  constexpr int GATES = C::GATES, NTW = C::NTW, R = C::R, UB = C::UB;
  constexpr bool BF = sizeof(T) == 2;
  constexpr int RP = R + 4;                       // LDS pitch of the gate tile (floats)
  constexpr int VE = 16 / sizeof(T);              // elements per 16-byte chunk
  constexpr int PAIRS = 16 * UB / kStepThreads;   // (batch row, unit) pairs per thread
  static_assert(PAIRS * kStepThreads == 16 * UB, "pairs");
  extern __shared__ __attribute__((aligned(16))) float step_smem[];
  float* gs = step_smem;                                        // [16][RP] gate pre-activations
  T* hs = reinterpret_cast<T*>(step_smem + 16 * RP);            // [16][H + VE] h_{t-1} rows

  const int H = p.hid, G = GATES * H, HP = H + VE;
  const int mdl = blockIdx.x / p.ublocks;
  const int ub = blockIdx.x - mdl * p.ublocks;
  const int u0 = ub * UB;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int fr = lane & 15, g = lane >> 4;
  const T* wb = static_cast<const T*>(p.w_hh) + static_cast<int64_t>(mdl) * G * H;
  const int nk = H / 32;

  for (int b0 = 0; b0 < p.batch; b0 += 16) {
    const T* wrow[NTW];
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      const int r = (wave * NTW + j) * 16 + fr;
      const int q = r / UB, u = u0 + (r - q * UB);
      wrow[j] = (u < H) ? wb + static_cast<int64_t>(q * H + u) * H + g * 8 : nullptr;
    }
    // (1) W_hh ring: PD k-steps of B fragments in flight (streams from L2 / MALL)
    constexpr int PD = BF ? 4 : 2;
    constexpr int BR = BF ? 1 : 2;                  // 16-byte pieces per fragment
    typedef typename std::conditional<BF, bf16x8, f32x4>::type frag_t;
    frag_t rb[PD][NTW][BR];
    auto ld = [&](frag_t (&b)[NTW][BR], int k) {
#pragma unroll
      for (int j = 0; j < NTW; ++j)
#pragma unroll
        for (int h2 = 0; h2 < BR; ++h2)
          b[j][h2] = wrow[j] ? *reinterpret_cast<const frag_t*>(wrow[j] + k * 32 + h2 * 4) : frag_t{};
    };
    if (p.hprev) {
#pragma unroll
      for (int s = 0; s < PD; ++s)
        if (s < nk) ld(rb[s], s);
    }
    // (2) the cell update's inputs, fetched now so they arrive during the K loop
    float gxv[PAIRS][GATES], cprev[PAIRS];
#pragma unroll
    for (int q = 0; q < PAIRS; ++q) {
      const int e = tid + q * kStepThreads;
      const int bl = e / UB, ul = e - (e / UB) * UB;
      const int b = b0 + bl, u = u0 + ul;
      const bool ok = b < p.batch && u < H;
      const int64_t nb = static_cast<int64_t>(mdl) * p.batch + b;
      const float* gxr = p.gx + (nb * p.steps + p.t) * G + u;
#pragma unroll
      for (int gi = 0; gi < GATES; ++gi) gxv[q][gi] = ok ? gxr[gi * H] : 0.f;
      cprev[q] = 0.f;
      if (CELL == WC_CELL_LSTM && ok)
        cprev[q] = p.t == 0 ? (p.c0 ? ldf<T>(p.c0, nb * H + u) : 0.f) : p.cst[nb * H + u];
    }
    // (3) h_{t-1} rows of this batch tile -> LDS (read once per workgroup)
    for (int c = tid; c < 16 * (H / VE); c += kStepThreads) {
      const int row = c / (H / VE), col = (c - row * (H / VE)) * VE;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (p.hprev && b0 + row < p.batch)
        v = *reinterpret_cast<const uint4*>(static_cast<const T*>(p.hprev) + mdl * p.hp_sn +
                                             static_cast<int64_t>(b0 + row) * p.hp_sb + col);
      *reinterpret_cast<uint4*>(hs + row * HP + col) = v;
    }
    __syncthreads();

    // (4) G = h_{t-1} W^T: 16 batch rows x R gate rows, A fragments from LDS
    f32x4 acc[NTW];
#pragma unroll
    for (int j = 0; j < NTW; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (p.hprev) {
      const T* arow = hs + fr * HP + g * 8;
      for (int k0 = 0; k0 < nk; k0 += PD) {
#pragma unroll
        for (int s = 0; s < PD; ++s) {
          if (k0 + s < nk) {
            const int k = k0 + s;
            if constexpr (BF) {
              const bf16x8 a = *reinterpret_cast<const bf16x8*>(arow + k * 32);
#pragma unroll
              for (int j = 0; j < NTW; ++j)
                acc[j] = mma16<T>(a, rb[s][j][0], acc[j]);
            } else {
              const f32x4 a0 = *reinterpret_cast<const f32x4*>(arow + k * 32);
              const f32x4 a1 = *reinterpret_cast<const f32x4*>(arow + k * 32 + 4);
#pragma unroll
              for (int j = 0; j < NTW; ++j) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                  acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[e], rb[s][j][0][e], acc[j], 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                  acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1[e], rb[s][j][1][e], acc[j], 0, 0, 0);
              }
            }
            if (k + PD < nk) ld(rb[s], k + PD);
          }
        }
      }
    }
    // lane holds G[b = (lane>>4)*4 + e][r = tile*16 + fr]
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      const int r = (wave * NTW + j) * 16 + fr;
#pragma unroll
      for (int e = 0; e < 4; ++e) gs[(g * 4 + e) * RP + r] = acc[j][e];
    }
    __syncthreads();

    // (5) cell update for this thread's (batch row, unit) pairs
#pragma unroll
    for (int q = 0; q < PAIRS; ++q) {
      const int e = tid + q * kStepThreads;
      const int bl = e / UB, ul = e - (e / UB) * UB;
      const int b = b0 + bl, u = u0 + ul;
      if (b >= p.batch || u >= H) continue;
      const int64_t nb = static_cast<int64_t>(mdl) * p.batch + b;
      const float* ghr = gs + bl * RP + ul;
      float gh[GATES];
#pragma unroll
      for (int gi = 0; gi < GATES; ++gi)
        gh[gi] = ghr[gi * UB] + (p.b_hh ? ldf<T>(p.b_hh, static_cast<int64_t>(mdl) * G + gi * H + u) : 0.f);
      float hnew, cnew = 0.f;
      if (CELL == WC_CELL_GRU) {
        const float hprev = to_f32(hs[bl * HP + u]);
        const float rg = sigmoid_f(gxv[q][0] + gh[0]);
        const float zg = sigmoid_f(gxv[q][1] + gh[1]);
        const float nn = tanh_f(gxv[q][2] + rg * gh[2]);
        hnew = (1.0f - zg) * nn + zg * hprev;
      } else {
        const float ig = sigmoid_f(gxv[q][0] + gh[0]);
        const float fg = sigmoid_f(gxv[q][1] + gh[1]);
        const float gg = tanh_f(gxv[q][2] + gh[2]);
        const float og = sigmoid_f(gxv[q][3] + gh[3]);
        cnew = fg * cprev[q] + ig * gg;
        hnew = og * tanh_f(cnew);
        p.cst[nb * H + u] = cnew;
      }
      static_cast<T*>(p.out)[(nb * p.steps + p.t) * H + u] = from_f32<T>(hnew);
      if (p.t == p.steps - 1) {
        if (p.hn) static_cast<T*>(p.hn)[nb * H + u] = from_f32<T>(hnew);
        if (CELL == WC_CELL_LSTM && p.cn) static_cast<T*>(p.cn)[nb * H + u] = from_f32<T>(cnew);
      }
    }
    __syncthreads();
  }
}

template <typename T, int CELL>
size_t step_lds_bytes(int hid) {
  using C = StepCfg<T, CELL>;
  return sizeof(float) * 16 * (C::R + 4) + sizeof(T) * 16 * static_cast<size_t>(hid + 16 / sizeof(T));
}

}  // namespace
}  // namespace wc

using namespace wc;

// Chooses the lane layout of the register-resident kernel; false when the
// weights of one (model, batch row) do not fit the register file.  Per step
// every SIMD issues, for each of its waves, the lane's GATES*UPG*KL FMAs,
// KL/4 LDS reads (each costed as 6 slots), GATES*UPG*log2(LG) DPP adds and a
// roughly fixed cell update (~60 issue slots with its transcendentals); the
// shape with the fewest slots on the busiest SIMD wins.  Weight registers stay
// <= 176 per lane (no spills).
static bool rnn_plan(int gates, int hid, RnnParams& p) {
  static const int kShapes[][3] = {   // {LG, UPG, KL}: the instantiated kernels
      {16, 1, 4}, {16, 2, 4}, {16, 4, 4}, {16, 1, 8}, {16, 2, 8}, {16, 4, 8}, {16, 1, 16}, {16, 2, 16},
      {16, 4, 16}, {8, 1, 4}, {8, 2, 4}, {8, 4, 4}, {8, 1, 8}, {8, 2, 8}, {8, 4, 8}, {8, 1, 16},
      {8, 2, 16}, {8, 4, 16}, {4, 1, 8}, {4, 2, 8}, {4, 1, 16}, {4, 2, 16}, {4, 1, 32}, {2, 1, 32}};
  long best = -1;
  for (const auto& sh : kShapes) {
    const int lg = sh[0], upg = sh[1], kl = sh[2];
    const int need = (hid + lg - 1) / lg;                    // columns per lane
    if (kl < need || (kl > 4 && kl / 2 >= need)) continue;   // the tightest instantiated KL only
    const int regs = gates * upg * kl;
    if (regs > 176) continue;
    const int threads = round_up(((hid + upg - 1) / upg) * lg, 64);
    if (threads > rnn_bound(gates, upg, kl)) continue;
    const int waves_per_simd = (threads / 64 + 3) / 4;
    int lg2 = 0;
    while ((1 << lg2) < lg) ++lg2;
    // LDS reads: a wave's 16-byte read moves 1 KB through the CU's shared LDS port, about
    // 6 VALU issue slots' worth of time (measured: for GRU H = 128, 8 lanes x 2 units x 16
    // columns runs 6% faster than 4 x 1 x 32, which a 1-slot read cost would have picked)
    const long cost = static_cast<long>(waves_per_simd) * (regs + 6 * (kl / 4) + gates * upg * lg2 + 60);
    if (best < 0 || cost < best) {
      best = cost;
      p.lg = lg;
      p.kl = kl;
      p.upg = upg;
    }
  }
  return best >= 0;
}

// every size in int32 range and every buffer of the problem (states, gates_x, x; counted in
// 8-byte elements) addressable in int64 bytes; the size arithmetic below runs only on such args
static bool rnn_sizes_fit(const wc_rnn_args* a) {
  const int64_t lim = 0x7fffffffll;
  if (a->n < 0 || a->batch < 0 || a->steps < 0 || a->hidden < 0 || a->input_size < 0) return false;
  if (a->n > lim || a->batch > lim || a->steps > lim || a->hidden > lim || a->input_size > lim) return false;
  int64_t nb, rows, e;
  if (__builtin_mul_overflow(a->n, a->batch, &nb) || __builtin_mul_overflow(nb, 4 * a->hidden, &e) ||
      __builtin_mul_overflow(e, int64_t{8}, &e))
    return false;                                    // h0 / c0 / h_n / c_n and the cell state
  if (__builtin_mul_overflow(nb, a->steps, &rows)) return false;
  if (__builtin_mul_overflow(rows, 4 * a->hidden, &e) || __builtin_mul_overflow(e, int64_t{8}, &e)) return false;
  if (__builtin_mul_overflow(rows, a->input_size, &e) || __builtin_mul_overflow(e, int64_t{8}, &e)) return false;
  return true;
}

static int64_t rnn_ws_bytes(const wc_rnn_args* a) {
  if (part_plan(a)) return part_workspace_bytes(a);
  const int64_t gates = a->cell == WC_CELL_GRU ? 3 : 4;
  // fp32 input projection [n, batch, steps, G] + fp32 cell state [n, batch, hidden]
  return (a->n * a->batch * a->steps * gates * a->hidden + a->n * a->batch * a->hidden) *
         static_cast<int64_t>(sizeof(float));
}

template <typename T, int CELL>
static int32_t streamed_recurrence(const wc_rnn_args* a, const RnnParams& rp, hipStream_t st) {
  using C = StepCfg<T, CELL>;
  StepParams p;
  p.n = rp.n;
  p.batch = rp.batch;
  p.steps = rp.steps;
  p.hid = rp.hid;
  p.ublocks = (rp.hid + C::UB - 1) / C::UB;
  p.gx = static_cast<const float*>(a->workspace);
  p.w_hh = a->w_hh;
  p.b_hh = a->b_hh;
  p.cst = static_cast<float*>(a->workspace) +
          static_cast<int64_t>(rp.n) * rp.batch * rp.steps * C::GATES * rp.hid;
  p.c0 = a->c0;
  p.out = a->out;
  p.hn = a->h_n;
  p.cn = a->c_n;
  const dim3 grid(static_cast<uint32_t>(static_cast<int64_t>(rp.n) * p.ublocks));
  const size_t lds = step_lds_bytes<T, CELL>(rp.hid);
  if (lds > 160 * 1024)
    return set_error(WC_ERR_LIMIT, "wc_rnn_recurrence: hidden=%d exceeds the streamed kernel's LDS", rp.hid);
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(rnn_step_kernel<T, CELL>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess)
      return set_error(static_cast<int32_t>(e), "wc_rnn_recurrence: LDS of %zu bytes refused: %s", lds,
                       hipGetErrorString(e));
  }
  for (int t = 0; t < rp.steps; ++t) {
    p.t = t;
    if (t == 0) {
      p.hprev = a->h0;
      p.hp_sn = static_cast<int64_t>(rp.batch) * rp.hid;
      p.hp_sb = rp.hid;
    } else {
      p.hprev = static_cast<const T*>(a->out) + static_cast<int64_t>(t - 1) * rp.hid;
      p.hp_sn = static_cast<int64_t>(rp.batch) * rp.steps * rp.hid;
      p.hp_sb = static_cast<int64_t>(rp.steps) * rp.hid;
    }
    rnn_step_kernel<T, CELL><<<grid, kStepThreads, lds, st>>>(p);
    int32_t rc = check_launch("wc_rnn_recurrence(step)");
    if (rc) return rc;
  }
  return WC_OK;
}

extern "C" int64_t wc_rnn_workspace_bytes(const wc_rnn_args* a) {
  if (!a || !rnn_sizes_fit(a)) return -1;
  return rnn_ws_bytes(a);
}

extern "C" int64_t wc_rnn_status_offset(const wc_rnn_args* a) {
  if (!a || !rnn_sizes_fit(a)) return -1;
  return part_plan(a) ? part_status_offset(a) : -1;
}

extern "C" int32_t wc_rnn_set_spin_limit(int32_t polls) { return part_set_spin_limit(polls); }

static int32_t rnn_check(const wc_rnn_args* a, const char* what, RnnParams& p, int& gates) {
  WC_REQUIRE(a != nullptr, WC_ERR_NULL, "%s: null args", what);
  WC_REQUIRE(a->cell == WC_CELL_GRU || a->cell == WC_CELL_LSTM, WC_ERR_ARG, "%s: unknown cell %d", what,
             a->cell);
  WC_REQUIRE(a->dtype == WC_F32 || a->dtype == WC_BF16 || a->dtype == WC_F16, WC_ERR_DTYPE,
             "%s: unsupported dtype %s", what, dtype_name(a->dtype));
  WC_REQUIRE(a->n >= 0 && a->batch >= 0 && a->steps >= 0 && a->input_size > 0 && a->hidden > 0,
             WC_ERR_SHAPE, "%s: bad sizes", what);
  gates = a->cell == WC_CELL_GRU ? 3 : 4;
  WC_REQUIRE(rnn_sizes_fit(a) && a->n * a->batch < 0x7fffffffll && a->batch * a->steps < 0x7fffffffll &&
                 gates * a->hidden < 0x7fffffffll,
             WC_ERR_LIMIT, "%s: sizes too large", what);
  p.n = (int)a->n;
  p.batch = (int)a->batch;
  p.steps = (int)a->steps;
  p.in = (int)a->input_size;
  p.hid = (int)a->hidden;
  if (p.n == 0 || p.batch == 0 || p.steps == 0) return WC_OK;
  WC_REQUIRE(a->workspace, WC_ERR_NULL, "%s: null workspace", what);
  WC_REQUIRE(a->workspace_bytes >= rnn_ws_bytes(a), WC_ERR_ARG, "%s: workspace of %lld bytes < %lld needed",
             what, (long long)a->workspace_bytes, (long long)rnn_ws_bytes(a));
  WC_REQUIRE(aligned(a->workspace, 16), WC_ERR_ALIGN, "%s: workspace not 16-byte aligned", what);
  WC_REQUIRE(aligned(a->status, 4), WC_ERR_ALIGN, "%s: status word not 4-byte aligned", what);
  return WC_OK;
}

extern "C" int32_t wc_rnn_input_projection(const wc_rnn_args* a, void* stream) {
  clear_error();
  RnnParams p;
  int gates = 0;
  int32_t rc = rnn_check(a, "wc_rnn_input_projection", p, gates);
  if (rc) return rc;
  if (p.n == 0 || p.batch == 0 || p.steps == 0) return WC_OK;
  WC_REQUIRE(a->x && a->w_ih, WC_ERR_NULL, "wc_rnn_input_projection: null pointer");
  const int G = gates * p.hid;
  const bool part = part_plan(a);
  void* bias_f32 = nullptr;
  if (part) {
    rc = part_prepare(a, as_stream(stream), &bias_f32);
    if (rc) return rc;
  }
  // gates_x = x W_ih^T + b_ih  ->  workspace [N, B*T, G]: fp32, or bf16 with b_ih + b_hh
  // folded in for the partitioned LSTM
  GemmParams g;
  g.n = p.n;
  g.m = p.batch * p.steps;
  g.o = G;
  g.k = p.in;
  g.act = WC_ACT_NONE;
  g.a = a->x;
  g.a_sn = a->x_stride_n;
  g.a_so = a->x_stride_b;
  g.a_si = a->x_stride_t;
  g.a_ri = make_fastdiv(static_cast<uint32_t>(p.steps));
  g.w = a->w_ih;
  g.w_sn = static_cast<int64_t>(G) * p.in;
  g.bias = a->b_ih;
  g.b_sn = G;
  g.r = nullptr;
  g.r_sn = g.r_so = g.r_si = 0;
  g.c = a->workspace;
  g.c_sn = static_cast<int64_t>(p.batch) * p.steps * G;
  g.c_so = 0;
  g.c_si = G;
  g.c_ri = make_fastdiv(static_cast<uint32_t>(p.batch * p.steps));
  if (part) {
    g.bias = bias_f32;
    return grouped_gemm(g, a->dtype, a->dtype, WC_F32, as_stream(stream));
  }
  return grouped_gemm(g, a->dtype, WC_F32, a->dtype, as_stream(stream));
}

// Launch the persistent kernel with the lane shape already in p (lg, kl, upg).
static int32_t persistent_recurrence(const wc_rnn_args* a, RnnParams p, int gates, hipStream_t st) {
  const int nwg = p.n * p.batch;
  p.remap = (nwg % 8 == 0) ? 1 : 0;
  p.gx = static_cast<const float*>(a->workspace);
  p.w_hh = a->w_hh;
  p.b_hh = a->b_hh;
  p.h0 = a->h0;
  p.c0 = a->c0;
  p.out = a->out;
  p.hn = a->h_n;
  p.cn = a->c_n;
  const int G = gates * p.hid;
  const size_t fixed = sizeof(float) * 2 * static_cast<size_t>(p.lg) * (p.kl + 4);
  const size_t per_step = sizeof(float) * static_cast<size_t>(G + p.hid);
  if (fixed + per_step > static_cast<size_t>(kRnnLdsBudget))
    return set_error(WC_ERR_LIMIT, "wc_rnn_recurrence: hidden=%d needs more LDS than available", p.hid);
  p.xt = static_cast<int>((kRnnLdsBudget - fixed) / per_step);
  if (p.xt > p.steps) p.xt = p.steps;
  const int threads = round_up(((p.hid + p.upg - 1) / p.upg) * p.lg, 64);
  const int es = dtype_size(a->dtype);
  p.wvec = (aligned(a->w_hh, 16) && ubytes(p.hid, es) % 16 == 0 && ubytes(p.kl, es) % 16 == 0) ? 1 : 0;
  const dim3 grid(nwg), block(threads);
  const size_t lds = fixed + per_step * static_cast<size_t>(p.xt);
  if (a->dtype == WC_F32) {
    if (a->cell == WC_CELL_GRU) return launch_rec<float, WC_CELL_GRU>(p, grid, block, lds, st);
    return launch_rec<float, WC_CELL_LSTM>(p, grid, block, lds, st);
  }
  if (a->dtype == WC_F16) {
    if (a->cell == WC_CELL_GRU) return launch_rec<f16, WC_CELL_GRU>(p, grid, block, lds, st);
    return launch_rec<f16, WC_CELL_LSTM>(p, grid, block, lds, st);
  }
  if (a->cell == WC_CELL_GRU) return launch_rec<bf16, WC_CELL_GRU>(p, grid, block, lds, st);
  return launch_rec<bf16, WC_CELL_LSTM>(p, grid, block, lds, st);
}

extern "C" int32_t wc_rnn_recurrence(const wc_rnn_args* a, void* stream) {
  clear_error();
  RnnParams p;
  int gates = 0;
  int32_t rc = rnn_check(a, "wc_rnn_recurrence", p, gates);
  if (rc) return rc;
  if (p.n == 0 || p.batch == 0 || p.steps == 0) return WC_OK;
  WC_REQUIRE(a->w_hh && a->out, WC_ERR_NULL, "wc_rnn_recurrence: null pointer");
  if (part_plan(a)) return part_recurrence(a, as_stream(stream));
  if (!rnn_plan(gates, p.hid, p)) {
    // W_hh of one model does not fit a workgroup's registers: one launch per step
    const int es = dtype_size(a->dtype);
    WC_REQUIRE(aligned(a->w_hh, 16) && ubytes(p.hid, es) % 16 == 0 && p.hid % 32 == 0 &&
                   (!a->h0 || aligned(a->h0, 16)) && aligned(a->out, 16),
               WC_ERR_ALIGN, "wc_rnn_recurrence: hidden=%d needs hidden %% 32 == 0 and 16-byte aligned "
               "W_hh / h0 / out for the streamed recurrence", p.hid);
    hipStream_t st = as_stream(stream);
    if (a->dtype == WC_F32)
      return a->cell == WC_CELL_GRU ? streamed_recurrence<float, WC_CELL_GRU>(a, p, st)
                                    : streamed_recurrence<float, WC_CELL_LSTM>(a, p, st);
    if (a->dtype == WC_F16)
      return a->cell == WC_CELL_GRU ? streamed_recurrence<f16, WC_CELL_GRU>(a, p, st)
                                    : streamed_recurrence<f16, WC_CELL_LSTM>(a, p, st);
    return a->cell == WC_CELL_GRU ? streamed_recurrence<bf16, WC_CELL_GRU>(a, p, st)
                                  : streamed_recurrence<bf16, WC_CELL_LSTM>(a, p, st);
  }
  return persistent_recurrence(a, p, gates, as_stream(stream));
}

extern "C" int32_t wc_rnn_forward(const wc_rnn_args* a, void* stream) {
  clear_error();
  RnnParams p;
  int gates = 0;
  int32_t rc = rnn_check(a, "wc_rnn_forward", p, gates);
  if (rc) return rc;
  if (p.n == 0 || p.batch == 0 || p.steps == 0) return WC_OK;
  rc = wc_rnn_input_projection(a, stream);
  if (rc) return rc;
  return wc_rnn_recurrence(a, stream);
}
