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

namespace wc {
namespace {

constexpr int kRnnMaxThreads = 1024;
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

// v_exp_f32 / v_rcp_f32 based activations, branch-free.  sigmoid has ~1e-7
// relative error; tanh(x) = 1 - 2 / (e^2x + 1) has ~1e-7 absolute error
// (its relative error grows only where |tanh| itself is below ~1e-3), both
// far inside the parity bars.
__device__ __forceinline__ float sigmoid_f(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

__device__ __forceinline__ float tanh_f(float x) {
  return 1.0f - 2.0f * __builtin_amdgcn_rcpf(__expf(2.0f * x) + 1.0f);
}

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

inline int round4(int v) { return (v + 3) & ~3; }
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
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, rb[s][j][0], acc[j], 0, 0, 0);
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

// ---------------------------------------------------------------------------
// Partitioned persistent LSTM recurrence (bf16; hidden 256, 384 or 512; batch <= 16).
//
// W_hh of one model (4H x H bf16: 2 MB at H = 512) exceeds one compute unit's
// registers and LDS, so P = H / 128 workgroups share a model, one per compute unit,
// for all T steps.  Workgroup `part` owns hidden units [128 part, 128 part + 128) and
// the 512 gate rows (i, f, g, o of each unit) of W_hh that feed them, held on-chip for
// the whole sequence: the first SL k-steps (32 columns each) in LDS, the rest in
// registers.  Per step it forms its gate pre-activations for all batch rows as MFMA
// tiles (A = W_hh rows, B = h_{t-1}^T read from LDS), applies the cell update in
// registers (the fp32 cell state never leaves the chip), writes h_t to the output,
// and publishes a per-(model, part) step counter; it then waits for the counters of
// the model's other parts and copies their slices of h_t into its LDS.
//
// Lane layout (v_mfma_f32_16x16x32_bf16, wave w of 4, lane = 16 g + fr): row tile j
// (0..7) of wave w holds A row rho = gate (rho & 3) of unit 32 w + 8 (rho >> 2) + j,
// so the accumulator of lane (g, fr) holds all four gates of unit 32 w + 8 g + j for
// batch row fr.  A lane therefore owns 8 consecutive units of one batch row: its
// gates_x of a gate, its h_t and its cell state are 16-byte vectors, and the cell
// update needs no data exchange between lanes.
//
// Cross-workgroup exchange.  h_t and the counters are written and read with
// device-scope (sc1) vector accesses, which are coherent across the XCDs' L2s; a
// part's h_t stores complete (vmcnt(0), then a barrier) before its counter is
// stored.  Counters sit in the caller's workspace: the input projection zeroes them,
// and the last workgroup of a model to finish resets them, so every launch starts
// from zero.  Every wait is bounded: past the limit the workgroup records 1 in the
// status word and leaves (the outputs are then invalid).  The host launches the grid
// cooperatively, so all workgroups are co-resident, or the launch fails.
// ---------------------------------------------------------------------------
constexpr int kPartUnits = 128;                      // hidden units per workgroup
constexpr int kPartThreads = 256;                    // 4 waves
constexpr int kPartSyncInts = 32;                    // one 128-byte block of counters per model
constexpr int kPartDone = 16;                        // index of the finished-parts counter
constexpr int kPartSpinLimit = 1 << 22;              // polls (each ~0.5 us) before giving up

struct PartParams {
  int n, batch, steps, remap;
  const bf16* gx;     // [n, batch, steps, 4H]: x W_ih^T + b_ih + b_hh, rounded to bf16
  const bf16* w_hh;   // [n, 4H, H]
  const bf16* h0;     // [n, batch, H] or null
  const bf16* c0;     // [n, batch, H] or null
  bf16* out;          // [n, batch, steps, H]
  bf16* hn;           // [n, batch, H] or null
  bf16* cn;           // [n, batch, H] or null
  int* sync;          // [n][kPartSyncInts] step counters and finished-parts counter
  int* status;        // set to 1 when a wait timed out
};

// k-steps of W_hh kept in LDS (the rest live in registers: 8 (16 - SL) fragments of
// 4 registers per lane at H = 512)
template <int H> struct PartCfg;
template <> struct PartCfg<256> { static constexpr int SL = 0; };
template <> struct PartCfg<384> { static constexpr int SL = 1; };
template <> struct PartCfg<512> { static constexpr int SL = 4; };

template <int H>
constexpr size_t part_lds_bytes() {
  return static_cast<size_t>(PartCfg<H>::SL) * 4 * 8 * 1024 + 16 * static_cast<size_t>(H + 8) * 2 + 16;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t part_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

constexpr int kSc1 = 16;   // buffer-op cache policy: device scope (sc1)

__device__ __forceinline__ int sync_load(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void sync_store(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int H>
__global__ __launch_bounds__(kPartThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void lstm_part_kernel(PartParams p) {
  constexpr int NT = 8, KS = H / 32, P = H / kPartUnits, SL = PartCfg<H>::SL, RS = KS - SL;
  constexpr int HP = H + 8;                          // LDS pitch of an h row (elements)
  constexpr int G = 4 * H;
  extern __shared__ __attribute__((aligned(16))) char part_smem[];
  bf16x8* wl = reinterpret_cast<bf16x8*>(part_smem);                          // [SL][4][NT][64]
  bf16* hs = reinterpret_cast<bf16*>(part_smem + SL * 4 * NT * 1024);         // [16][HP] h_{t-1}
  int* abort_flag = reinterpret_cast<int*>(hs + 16 * HP);

  const int nwg = p.n * P;
  int id = blockIdx.x;
  if (p.remap) id = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);   // a model's parts share an XCD
  const int mdl = id / P, part = id - mdl * P;
  const int u0 = part * kPartUnits;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, fr = lane & 15;
  const int ucol = u0 + w * 32 + g * 8;              // first of the lane's 8 units (model column)
  const bool brow = fr < p.batch;
  const int64_t mb = static_cast<int64_t>(mdl) * p.batch;

  // ---- W_hh rows of this part: registers and LDS, loaded once ----
  bf16x8 wr[RS > 0 ? RS : 1][NT];
  {
    const bf16* wb = p.w_hh + static_cast<int64_t>(mdl) * G * H;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const bf16* row = wb + static_cast<int64_t>((fr & 3) * H + u0 + w * 32 + (fr >> 2) * 8 + j) * H + g * 8;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const bf16x8 v = *reinterpret_cast<const bf16x8*>(row + s * 32);
        if (s < SL) wl[((s * 4 + w) * NT + j) * 64 + lane] = v;
        else wr[s - SL][j] = v;
      }
    }
  }
  // ---- h_{-1} into LDS (rows >= batch stay zero), c_{-1} and gates_x of step 0 in registers ----
  for (int e = tid; e < 16 * (HP / 8); e += kPartThreads) {
    const int b = e / (HP / 8), col = (e - b * (HP / 8)) * 8;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (p.h0 && b < p.batch && col < H)
      v = *reinterpret_cast<const uint4*>(p.h0 + (mb + b) * H + col);
    *reinterpret_cast<uint4*>(hs + b * HP + col) = v;
  }
  if (tid == 0) *abort_flag = 0;
  float c[NT];
  {
    bf16x8 cv = {};
    if (p.c0 && brow) cv = *reinterpret_cast<const bf16x8*>(p.c0 + (mb + fr) * H + ucol);
#pragma unroll
    for (int j = 0; j < NT; ++j) c[j] = static_cast<float>(cv[j]);
  }
  const uint32_t out_bytes = static_cast<uint32_t>(p.batch) * p.steps * H * 2;   // this model's out block
  const __amdgpu_buffer_rsrc_t ors = part_rsrc(p.out + mb * p.steps * H, out_bytes);
  const __amdgpu_buffer_rsrc_t grs =
      part_rsrc(p.gx + mb * p.steps * G, static_cast<uint32_t>(p.batch) * p.steps * G * 2);
  const uint32_t lane_row = static_cast<uint32_t>(brow ? fr : 0) * p.steps;   // (b * steps) for this lane
  bf16x8 gxn[4];
  auto load_gx = [&](int t) {
    const uint32_t off = ((lane_row + t) * G + ucol) * 2;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      gxn[q] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(grs, off + q * H * 2, 0, 0));
  };
  load_gx(0);
  int* my_sync = p.sync + static_cast<int64_t>(mdl) * kPartSyncInts;
  __syncthreads();

  bool aborted = false;
  bf16x8 hv = {};
  for (int t = 0; t < p.steps; ++t) {
    // gates = gates_x (incl. both biases) + h_{t-1} W_hh^T
    f32x4 acc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[j][e] = static_cast<float>(gxn[e][j]);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const bf16x8 hb = *reinterpret_cast<const bf16x8*>(hs + fr * HP + s * 32 + g * 8);
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const bf16x8 a = (s < SL) ? wl[((s * 4 + w) * NT + j) * 64 + lane] : wr[s < SL ? 0 : s - SL][j];
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, hb, acc[j], 0, 0, 0);
      }
    }
    // cell update of the lane's 8 units (i, f, g, o in acc[j][0..3])
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const float ig = sigmoid_f(acc[j][0]);
      const float fg = sigmoid_f(acc[j][1]);
      const float gg = tanh_f(acc[j][2]);
      const float og = sigmoid_f(acc[j][3]);
      c[j] = fg * c[j] + ig * gg;
      hv[j] = static_cast<bf16>(og * tanh_f(c[j]));
    }
    if (brow)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, hv), ors,
                                             ((lane_row + t) * H + ucol) * 2, 0, kSc1);
    if (t + 1 == p.steps) break;
    __syncthreads();                                   // every wave has read h_{t-1}
    *reinterpret_cast<bf16x8*>(hs + fr * HP + ucol) = hv;
    if (P > 1) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's h_t stores are performed
      __syncthreads();
      if (tid == 0) sync_store(my_sync + part, t + 1);
    }
    load_gx(t + 1);
    if (P > 1) {
      if (w == 0) {
        bool ok = true;
        if (lane < P && lane != part) {
          int spins = 0;
          while (sync_load(my_sync + lane) < t + 1) {
            if (++spins > kPartSpinLimit) {
              ok = false;
              break;
            }
            __builtin_amdgcn_s_sleep(2);
          }
        }
        if (!ok) *abort_flag = 1;
      }
      __syncthreads();
      if (*abort_flag) {
        aborted = true;
        break;
      }
      // the other parts' slices of h_t: rows < batch, 128-unit slices != part
      constexpr int CH = (P - 1) * (kPartUnits / 8);   // 16-byte chunks per row
      for (int e = tid; e < p.batch * CH; e += kPartThreads) {
        const int b = e / CH, r = e - b * CH;
        int q = r / (kPartUnits / 8);
        q += (q >= part) ? 1 : 0;
        const int col = q * kPartUnits + (r % (kPartUnits / 8)) * 8;
        const i32x4 v = __builtin_amdgcn_raw_buffer_load_b128(
            ors, ((static_cast<uint32_t>(b) * p.steps + t) * H + col) * 2, 0, kSc1);
        *reinterpret_cast<i32x4*>(hs + b * HP + col) = v;
      }
    }
    __syncthreads();
  }

  if (!aborted && brow) {
    const int64_t so = (mb + fr) * H + ucol;
    if (p.hn) *reinterpret_cast<bf16x8*>(p.hn + so) = hv;
    if (p.cn) {
      bf16x8 cv;
#pragma unroll
      for (int j = 0; j < NT; ++j) cv[j] = static_cast<bf16>(c[j]);
      *reinterpret_cast<bf16x8*>(p.cn + so) = cv;
    }
  }
  if (P > 1) {
    // the last part of the model to finish resets the counters for the next launch
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      if (aborted) sync_store(p.status, 1);
      const int before = __hip_atomic_fetch_add(my_sync + kPartDone, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (before == P - 1) {
#pragma unroll
        for (int q = 0; q < P; ++q) sync_store(my_sync + q, 0);
        sync_store(my_sync + kPartDone, 0);
      }
    }
  }
}

// counters and status zeroed; bias = b_ih + b_hh in fp32 (either may be null)
__global__ void part_prep_kernel(int* sync, int nsync, const bf16* b_ih, const bf16* b_hh, float* bias,
                                 int64_t nbias) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < nsync) sync_store(sync + i, 0);
  if (bias && i < nbias)
    bias[i] = (b_ih ? static_cast<float>(b_ih[i]) : 0.f) + (b_hh ? static_cast<float>(b_hh[i]) : 0.f);
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

// ---- partitioned LSTM: when it applies, and its workspace layout ----
template <int H>
static bool part_kernel_fits(size_t& lds) {
  lds = part_lds_bytes<H>();
  const void* fn = reinterpret_cast<const void*>(lstm_part_kernel<H>);
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) != hipSuccess)
    return false;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kPartThreads, lds) != hipSuccess) return false;
  return per_cu >= 1;
}

// The partitioned kernel runs bf16 LSTMs with hidden 256 / 384 / 512 and batch <= 16 when
// every (model, part) workgroup can hold a compute unit of its own.
static bool part_plan(const wc_rnn_args* a) {
  if (a->cell != WC_CELL_LSTM || a->dtype != WC_BF16 || a->batch < 1 || a->batch > 16 || a->steps < 1)
    return false;
  if (a->hidden != 256 && a->hidden != 384 && a->hidden != 512) return false;
  const int64_t parts = a->hidden / kPartUnits;
  const int cus = device_cu_count();
  if (cus <= 0 || a->n * parts > cus) return false;
  // per-model blocks of gates_x and out are addressed with 32-bit byte offsets
  if (a->batch * a->steps * 4 * a->hidden * 2 >= 0x7fffffffll) return false;
  for (const void* q : {a->w_hh, a->h0, a->c0, static_cast<const void*>(a->out),
                        static_cast<const void*>(a->h_n), static_cast<const void*>(a->c_n)})
    if (q && !aligned(q, 16)) return false;
  size_t lds = 0;
  if (a->hidden == 256) return part_kernel_fits<256>(lds);
  if (a->hidden == 384) return part_kernel_fits<384>(lds);
  return part_kernel_fits<512>(lds);
}

inline int64_t round256(int64_t v) { return (v + 255) & ~static_cast<int64_t>(255); }

struct PartLayout {
  int64_t gx, bias, sync, status, total;   // byte offsets into the workspace
};

static PartLayout part_layout(const wc_rnn_args* a) {
  const int64_t g = 4 * a->hidden;
  PartLayout l;
  l.gx = 0;
  l.bias = round256(a->n * a->batch * a->steps * g * 2);
  l.sync = l.bias + round256(a->n * g * 4);
  l.status = l.sync + round256(a->n * kPartSyncInts * 4);
  l.total = l.status + 256;
  return l;
}

static int64_t rnn_ws_bytes(const wc_rnn_args* a) {
  if (part_plan(a)) return part_layout(a).total;
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
  if (!a || a->n < 0 || a->batch < 0 || a->steps < 0 || a->hidden < 0) return -1;
  return rnn_ws_bytes(a);
}

extern "C" int64_t wc_rnn_status_offset(const wc_rnn_args* a) {
  if (!a || a->n < 0 || a->batch < 0 || a->steps < 0 || a->hidden < 0) return -1;
  return part_plan(a) ? part_layout(a).status : -1;
}

static int32_t rnn_check(const wc_rnn_args* a, const char* what, RnnParams& p, int& gates) {
  WC_REQUIRE(a != nullptr, WC_ERR_NULL, "%s: null args", what);
  WC_REQUIRE(a->cell == WC_CELL_GRU || a->cell == WC_CELL_LSTM, WC_ERR_ARG, "%s: unknown cell %d", what,
             a->cell);
  WC_REQUIRE(a->dtype == WC_F32 || a->dtype == WC_BF16, WC_ERR_DTYPE, "%s: unsupported dtype %s", what,
             dtype_name(a->dtype));
  WC_REQUIRE(a->n >= 0 && a->batch >= 0 && a->steps >= 0 && a->input_size > 0 && a->hidden > 0,
             WC_ERR_SHAPE, "%s: bad sizes", what);
  gates = a->cell == WC_CELL_GRU ? 3 : 4;
  WC_REQUIRE(a->n * a->batch < 0x7fffffffll && a->batch * a->steps < 0x7fffffffll &&
                 gates * a->hidden < 0x7fffffffll && a->input_size < 0x7fffffffll,
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
    // zero the step counters and status word; bias = b_ih + b_hh (fp32) for the projection
    const PartLayout l = part_layout(a);
    char* ws = static_cast<char*>(a->workspace);
    const int nsync = static_cast<int>((l.total - l.sync) / 4);
    const int64_t nbias = (a->b_ih || a->b_hh) ? static_cast<int64_t>(p.n) * G : 0;
    if (nbias) bias_f32 = ws + l.bias;
    const int64_t items = nbias > nsync ? nbias : nsync;
    part_prep_kernel<<<static_cast<uint32_t>(cdiv(items, 256)), 256, 0, as_stream(stream)>>>(
        reinterpret_cast<int*>(ws + l.sync), nsync, static_cast<const bf16*>(a->b_ih),
        static_cast<const bf16*>(a->b_hh), static_cast<float*>(bias_f32), nbias);
    rc = check_launch("wc_rnn_input_projection(prep)");
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

template <int H>
static int32_t launch_part(const wc_rnn_args* a, hipStream_t st) {
  const PartLayout l = part_layout(a);
  char* ws = static_cast<char*>(a->workspace);
  PartParams p;
  p.n = static_cast<int>(a->n);
  p.batch = static_cast<int>(a->batch);
  p.steps = static_cast<int>(a->steps);
  const int nwg = p.n * (H / kPartUnits);
  p.remap = (nwg % 8 == 0 && (nwg / 8) % (H / kPartUnits) == 0) ? 1 : 0;
  p.gx = reinterpret_cast<const bf16*>(ws + l.gx);
  p.w_hh = static_cast<const bf16*>(a->w_hh);
  p.h0 = static_cast<const bf16*>(a->h0);
  p.c0 = static_cast<const bf16*>(a->c0);
  p.out = static_cast<bf16*>(a->out);
  p.hn = static_cast<bf16*>(a->h_n);
  p.cn = static_cast<bf16*>(a->c_n);
  p.sync = reinterpret_cast<int*>(ws + l.sync);
  p.status = reinterpret_cast<int*>(ws + l.status);
  const size_t lds = part_lds_bytes<H>();
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cap) != hipSuccess)
    return set_error(WC_ERR_ARG, "wc_rnn_recurrence: stream capture status unavailable");
  if (cap == hipStreamCaptureStatusNone) {
    // co-residency of the whole grid is guaranteed, or the launch fails here
    void* args[] = {&p};
    const hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(lstm_part_kernel<H>),
                                                    dim3(nwg), dim3(kPartThreads), args,
                                                    static_cast<unsigned>(lds), st);
    if (e != hipSuccess)
      return set_error(static_cast<int32_t>(e), "wc_rnn_recurrence: cooperative launch of %d workgroups "
                       "failed: %s", nwg, hipGetErrorString(e));
    return WC_OK;
  }
  // under graph capture: an ordinary kernel node (the host checked that the grid fits the
  // device one workgroup per compute unit)
  lstm_part_kernel<H><<<dim3(nwg), dim3(kPartThreads), lds, st>>>(p);
  return check_launch("wc_rnn_recurrence(partitioned)");
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
  p.wvec = (aligned(a->w_hh, 16) && (p.hid * es) % 16 == 0 && (p.kl * es) % 16 == 0) ? 1 : 0;
  const dim3 grid(nwg), block(threads);
  const size_t lds = fixed + per_step * static_cast<size_t>(p.xt);
  if (a->dtype == WC_F32) {
    if (a->cell == WC_CELL_GRU) return launch_rec<float, WC_CELL_GRU>(p, grid, block, lds, st);
    return launch_rec<float, WC_CELL_LSTM>(p, grid, block, lds, st);
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
  if (part_plan(a)) {
    hipStream_t st = as_stream(stream);
    if (p.hid == 256) return launch_part<256>(a, st);
    if (p.hid == 384) return launch_part<384>(a, st);
    return launch_part<512>(a, st);
  }
  if (!rnn_plan(gates, p.hid, p)) {
    // W_hh of one model does not fit a workgroup's registers: one launch per step
    const int es = dtype_size(a->dtype);
    WC_REQUIRE(aligned(a->w_hh, 16) && (p.hid * es) % 16 == 0 && p.hid % 32 == 0 &&
                   (!a->h0 || aligned(a->h0, 16)) && aligned(a->out, 16),
               WC_ERR_ALIGN, "wc_rnn_recurrence: hidden=%d needs hidden %% 32 == 0 and 16-byte aligned "
               "W_hh / h0 / out for the streamed recurrence", p.hid);
    hipStream_t st = as_stream(stream);
    if (a->dtype == WC_F32)
      return a->cell == WC_CELL_GRU ? streamed_recurrence<float, WC_CELL_GRU>(a, p, st)
                                    : streamed_recurrence<float, WC_CELL_LSTM>(a, p, st);
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
