// Partitioned persistent recurrence: LSTM and GRU, bf16 or fp16, hidden 256, 384 or 512.
//
// W_hh of one model (G x H 16-bit values, G = 4H for the LSTM: 2 MB at H = 512) exceeds one
// compute unit's registers and LDS, so P = H / 128 workgroups share a model, one per compute
// unit, for all T steps.  Workgroup `part` owns hidden units [128 part, 128 part + 128) and
// the gate rows of W_hh that feed them, held on-chip for the whole sequence, k-step by
// k-step (32 columns each) in storage slots: the first SL slots in LDS, the next NA in AGPRs
// (loaded there directly and read in place as MFMA A operands), the rest in VGPRs; k-step k
// sits in slot (k + SH) % KS, where the LSTM's SH = SL puts its own k-steps in registers.
// This file is built with -amdgpu-mfma-vgpr-form so that accumulators live in VGPRs and the
// AGPR file is left to the weights.
//
// The work is split into units of (model, chunk of up to 16 batch rows): batch rows of a
// recurrence are independent, so a chunk has its own cell state, exchange slots and step
// counters.  One launch runs up to (compute units / P) units; more units take several
// launches in a row on the stream.
//
// Per step a workgroup forms its gate pre-activations for the chunk's rows as MFMA tiles
// (A = W_hh rows, B = h_{t-1}^T read from LDS; the LSTM's accumulators start from gates_x,
// the GRU adds gates_x in the cell update), applies the cell update in registers (the
// fp32 state -- the LSTM cell state, the GRU hidden state -- never leaves the chip), writes
// h_t to the output and to an exchange slot, and copies the other parts' slices of h_t from
// their exchange slots into its LDS.
//
// Lane layout (v_mfma_f32_16x16x32 on 16-bit operands, wave w of 4, lane = 16 g + fr): row
// tile j (0..7) of wave w holds A row rho = gate slot (rho & 3) of unit 32 w + 8 (rho >> 2)
// + j, so the accumulator of lane (g, fr) holds the four gate slots of unit 32 w + 8 g + j
// for chunk row fr.  LSTM slots are the gates i, f, g, o; GRU slots are r, z, n and a fourth
// whose W rows repeat those of n and whose result is never read.  A lane therefore owns 8
// consecutive units of one row: its gates_x of a gate, its h_t and its state are 16-byte
// vectors, and the cell update needs no data exchange between lanes.
//
// Exchange.  Every exchanged value carries the step it belongs to, so a reader polls the
// values it needs with device-scope (sc1) loads until every tag matches, and no separate
// flag, store fence or extra round trip is needed.  LSTM: h = o tanh(c) lies in [-1, 1], so
// bit 14 of its 16-bit form (the top exponent bit) is free and holds a 1-bit tag; the values
// travel 8 to a 16-byte chunk.  GRU (whose h follows h0, which may exceed 1): each value is
// one 32-bit word, (16 bits of h << 16) | tag with a 16-bit tag.  Under load the exchange
// costs in proportion to its bytes (the LSTM form halved a c5 step's poll round, 3.5k ->
// 1.6k cycles).  Writers use device-scope stores too, unless every part of the unit runs on
// one XCD (read from HW_REG_XCC_ID at start), in which case plain stores into the shared L2
// suffice and are faster.  There are two slots per unit (step parity): a part cannot write
// step t + 2 into a slot before every other part has read step t from it, since it needs
// their step t + 1 first.  `base` lives in the caller's workspace: the input projection
// zeroes it and fills the slots with all-ones words (word tag 0xFFFF, bit 14 set in every
// 16-bit half), and the last workgroup of a unit to finish advances it by T.  So a stale
// LSTM value is always exactly 2 steps old (every step is published, the last one of a launch
// included, and the tag base is 16 bits wide, a multiple of the tag's period 4), and a stale
// GRU word 1 or 2 steps behind the one a reader expects.  Every wait is bounded: past the
// limit (poll rounds, set by the host; 0 gives up at the first wait without polling) the
// workgroup records 1 in the status word and leaves
// (the outputs are then invalid).  The status word is the caller's own when one is passed
// (never cleared here), else a word of the workspace that the input projection zeroes.  The
// host launches the grid cooperatively, so all workgroups are co-resident or the launch
// fails.
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <type_traits>

#include "wc_rnn.h"

namespace wc {
namespace {

constexpr int kPartUnits = 128;        // hidden units per workgroup
constexpr int kPartThreads = 256;      // 4 waves
constexpr int kSyncInts = 32;          // one 128-byte block per model:
constexpr int kSyncDone = 16;          //   finished-parts counter
constexpr int kSyncBase = 17;          //   tag of this launch's step 0
constexpr int kSyncXcc = 20;           //   per part: (tag of step 0 << 16) | (XCD + 1)
constexpr int kSpinLimit = 1 << 21;    // default poll rounds (each >= ~0.5 us) before giving up
constexpr int kSc1 = 16;               // buffer-op cache policy: device scope (sc1)
constexpr uint32_t kTagFill = 0xFFFFFFFFu;  // word tag 0xFFFF; both halves with bit 14 set

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

struct PartParams {
  int n, rows, chunks;  // models, batch rows, 16-row chunks per model
  int unit0, steps, remap;
  int spin_limit;       // poll rounds of a wait before it gives up (0: at once)
  const void* gx;       // [n, rows, steps, G]: x W_ih^T + folded biases, in the element type
  const void* w_hh;     // [n, G, H]
  const void* h0;       // [n, rows, H] or null
  const void* c0;       // LSTM: [n, rows, H] or null
  const float* bhn;     // GRU: [n, H] fp32 b_hh of gate n, or null
  void* out;            // [n, rows, steps, H]
  void* hn;             // [n, rows, H] or null
  void* cn;             // LSTM: [n, rows, H] or null
  uint32_t* xch;        // [units][2][16][H] exchange words (LSTM: 16-bit values in the first half)
  int* sync;            // [units][kSyncInts]
  int* status;          // set to 1 when a wait gave up
};

std::atomic<int> g_spin_limit{kSpinLimit};

// Where the (storage slot q, row tile j) fragments of W_hh live: q < SL in LDS, q < SL + NA
// in AGPRs, tiles j < XL of slot SL + NA in LDS as well, the rest in VGPRs.  k-step k (in the
// rotated order, this part's own columns first) is kept in slot (k + SH) % KS.  The LSTM
// takes SH = SL, so its own k-steps are register-fed: they run between the exchange store and
// the exchange poll, where nothing hides an LDS read per MFMA, while the non-own k-steps run
// beside the cell update (1-2 % per step); the GRU keeps SH = 0 (with SH = SL its H = 512
// form spills).
template <int H> struct PartCfg;
template <> struct PartCfg<256> { static constexpr int SL = 0, NA = 6, XL = 0; };
template <> struct PartCfg<384> { static constexpr int SL = 1, NA = 8, XL = 0; };
template <> struct PartCfg<512> { static constexpr int SL = 4, NA = 8, XL = 3; };

// The order in which the k-steps B..E-1 are visited (s: k-step, q: its storage slot):
// LDS-fed k-steps (q < SL, and SL + NA when XL > 0) alternate with register-fed ones, so the
// fragments of the next LDS-fed k-step are read while the MFMAs of a register-fed k-step run.
template <int SL, int NA, int XL, int KS, int SH, int B, int E>
struct KOrder {
  int s[E - B], q[E - B];
  bool lds[E - B];
  constexpr KOrder() : s(), q(), lds() {
    int ls[E - B] = {}, rs[E - B] = {};
    int nl = 0, nr = 0;
    for (int k = B; k < E; ++k) {
      const int qk = (k + SH) % KS;
      if (qk < SL || (XL > 0 && qk == SL + NA)) ls[nl++] = k;
      else rs[nr++] = k;
    }
    int o = 0, il = 0, ir = 0;
    while (il < nl || ir < nr) {
      if (il < nl) { s[o] = ls[il++]; lds[o++] = true; }
      if (ir < nr) { s[o] = rs[ir++]; lds[o++] = false; }
    }
    for (int i = 0; i < E - B; ++i) q[i] = (s[i] + SH) % KS;
  }
};

// acc[j] += the k-steps B..E-1 of (W_hh rows of tile j) x h^T for the tiles J0 <= j < J1:
// A fragments from LDS (wlw, this lane's fragment base), AGPRs (wa) or VGPRs (wv); B fragments
// from this lane's h row in LDS (hrow, k-step s at hrow + 32 s).
template <typename T, int SL, int NA, int XL, int KS, int SH, int B, int E, int J0, int J1, int NT, int RA,
          int RV>
__device__ __forceinline__ void mfma_steps(f32x4 (&acc)[NT], const bf16x8 (&wa)[RA][NT],
                                           const bf16x8 (&wv)[RV][NT], const bf16x8* wlw, const bf16* hrow) {
  static_assert(0 <= J0 && J0 < J1 && J1 <= NT, "tile range");
  constexpr KOrder<SL, NA, XL, KS, SH, B, E> ord;
  constexpr int N = E - B;
  bf16x8 lf[NT];                                     // LDS-fed fragments of the current / next k-step
  auto in_lds = [](int q, int j) { return q < SL || (XL > 0 && q == SL + NA && j < XL); };
  auto load_tile = [&](int q, int j) {
    if (q < SL) lf[j] = wlw[(q * NT + j) * 64];
    else if (in_lds(q, j)) lf[j] = wlw[(SL * NT + j) * 64];
  };
  bf16x8 hb = *reinterpret_cast<const bf16x8*>(hrow + ord.s[0] * 32);
  if (ord.lds[0]) {
#pragma unroll
    for (int j = J0; j < J1; ++j) load_tile(ord.q[0], j);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int q = ord.q[i];
    const bool nxt_lds = i + 1 < N && ord.lds[i + 1];
    const bf16x8 hc = hb;
    if (i + 1 < N) hb = *reinterpret_cast<const bf16x8*>(hrow + ord.s[i + 1] * 32);
    // a register-fed k-step: read all of the next LDS-fed k-step's fragments under its MFMAs
    if (!ord.lds[i] && nxt_lds) {
#pragma unroll
      for (int j = J0; j < J1; ++j) load_tile(ord.q[i + 1], j);
    }
#pragma unroll
    for (int j = J0; j < J1; ++j) {
      bf16x8 a;
      if (in_lds(q, j)) a = lf[j];
      else if (q < SL + NA) a = wa[q < SL + NA ? q - SL : 0][j];
      else a = wv[q < SL + NA ? 0 : q - SL - NA][j];
      acc[j] = mma16<T>(a, hc, acc[j]);
      // two LDS-fed k-steps in a row: refill tile j once its MFMA has taken it
      if (ord.lds[i] && nxt_lds) load_tile(ord.q[i + 1], j);
    }
  }
}

template <int H>
constexpr size_t part_lds_bytes() {
  return (static_cast<size_t>(PartCfg<H>::SL) * 8 + PartCfg<H>::XL) * 4 * 1024 +
         16 * static_cast<size_t>(H + 8) * 2 + 16;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t part_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// element j of 8 raw 16-bit lanes of type T, as float; store a float there, rounded
template <typename T>
__device__ __forceinline__ float lane_f(const bf16x8& v, int j) {
  if constexpr (std::is_same<T, f16>::value) return static_cast<float>(__builtin_bit_cast(f16x8, v)[j]);
  else return static_cast<float>(v[j]);
}
template <typename T>
__device__ __forceinline__ void set_lane(bf16x8& v, int j, float x) {
  if constexpr (std::is_same<T, f16>::value) {
    f16x8 t = __builtin_bit_cast(f16x8, v);
    t[j] = static_cast<f16>(x);
    v = __builtin_bit_cast(bf16x8, t);
  } else {
    v[j] = static_cast<bf16>(x);
  }
}

// gates i, f, g, o of the lane's unit j from the four gates_x vectors, as an accumulator
template <typename T>
__device__ __forceinline__ f32x4 gx_acc(const bf16x8* gx, int j) {
  return f32x4{lane_f<T>(gx[0], j), lane_f<T>(gx[1], j), lane_f<T>(gx[2], j), lane_f<T>(gx[3], j)};
}

// LDS-only barrier: waits for this wave's LDS traffic, not for its global loads and
// stores, which stay in flight across it
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ int sync_load(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void sync_store(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int H, typename T, int CELL>
__global__ __launch_bounds__(kPartThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void part_kernel(PartParams p) {
  constexpr bool GRU = CELL == WC_CELL_GRU;
  constexpr int NT = 8, KS = H / 32, P = H / kPartUnits;
  constexpr int SL = PartCfg<H>::SL, NA = PartCfg<H>::NA, XL = PartCfg<H>::XL, NV = KS - SL - NA;
  static_assert(NV >= 0 && P >= 2, "partition");
  constexpr int SH = GRU ? 0 : SL;                   // W_hh storage slot of k-step k: (k + SH) % KS
  constexpr int HP = H + 8;                          // LDS pitch of an h row (elements)
  constexpr int G = (GRU ? 3 : 4) * H;
  constexpr int NG = GRU ? 3 : 4;                    // gates_x vectors a lane reads per step
  constexpr int KPP = kPartUnits / 32;               // k-steps of one part's columns
  constexpr int CPR = (P - 1) * kPartUnits / 4;      // remote 16-byte exchange chunks per row
  constexpr int CPT = (16 * CPR + kPartThreads - 1) / kPartThreads;
  extern __shared__ __attribute__((aligned(16))) char part_smem[];
  // LDS-resident W_hh fragments, [wave][f][64 lanes] x 16 bytes, f = 8 s + j for s < SL and
  // 8 SL + j for the XL tiles of k-step SL + NA: one wave's fragments lie within 64 KB of
  // its base, so every read is the base plus an immediate offset
  constexpr int NF = SL * NT + XL;
  bf16x8* wl = reinterpret_cast<bf16x8*>(part_smem);
  bf16* hs = reinterpret_cast<bf16*>(part_smem + (SL * NT + XL) * 4 * 1024);  // [16][HP] h_{t-1} (raw 16-bit)
  int* abort_flag = reinterpret_cast<int*>(hs + 16 * HP);
  int* xcd_flag = abort_flag + 1;

  const int nwg = static_cast<int>(gridDim.x);
  int id = blockIdx.x;
  if (p.remap) id = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);   // a unit's parts share an XCD
  const int lu = id / P, part = id - lu * P;
  const int unit = p.unit0 + lu;                     // (model, chunk) of this workgroup
  const int mdl = unit / p.chunks, chk = unit - mdl * p.chunks;
  const int row0 = chk * 16;
  const int nrows = p.rows - row0 < 16 ? p.rows - row0 : 16;
  const int u0 = part * kPartUnits;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, fr = lane & 15;
  const int ucol = u0 + w * 32 + g * 8;              // first of the lane's 8 units (model column)
  const bool brow = fr < nrows;
  const int64_t mb = static_cast<int64_t>(mdl) * p.rows + row0;   // the chunk's first row
  const bf16* const h0 = static_cast<const bf16*>(p.h0);
  const bf16* const c0 = static_cast<const bf16*>(p.c0);

  // ---- W_hh rows of this part in LDS, AGPRs and VGPRs, loaded once (GRU: gate slot 3
  // repeats the n rows; its accumulator is never read) ----
  bf16x8 wa[NA > 0 ? NA : 1][NT];
  bf16x8 wv[NV > 0 ? NV : 1][NT];
  {
    const bf16* wb = static_cast<const bf16*>(p.w_hh) + static_cast<int64_t>(mdl) * G * H;
    const int slot = GRU && (fr & 3) == 3 ? 2 : (fr & 3);
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const bf16* row = wb + static_cast<int64_t>(slot * H + u0 + w * 32 + (fr >> 2) * 8 + j) * H + g * 8;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const bf16* src = row + ((s + KS - SH + part * KPP) % KS) * 32;   // slot s: rotated k-step s - SH
        if (s < SL) {
          wl[(w * NF + s * NT + j) * 64 + lane] = *reinterpret_cast<const bf16x8*>(src);
        } else if (s < SL + NA) {
          asm volatile("global_load_dwordx4 %0, %1, off" : "=a"(wa[s - SL][j]) : "v"(src));
        } else if (s == SL + NA && j < XL) {
          wl[(w * NF + SL * NT + j) * 64 + lane] = *reinterpret_cast<const bf16x8*>(src);
        } else {
          wv[s - SL - NA][j] = *reinterpret_cast<const bf16x8*>(src);
        }
      }
    }
    // the AGPR loads are invisible to the compiler's wait counting: wait here, and make
    // every later use of those registers depend on this point
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int i = 0; i < NA; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) asm volatile("" : "+a"(wa[i][j]));
  }
  // ---- h_{-1} into LDS (rows >= nrows stay zero); the state (LSTM: c_{-1}, GRU: h_{-1}) and
  // gates_x of step 0 in registers ----
  for (int e = tid; e < 16 * (HP / 8); e += kPartThreads) {
    const int b = e / (HP / 8), col = (e - b * (HP / 8)) * 8;   // LDS column (rotated)
    uint4 v = make_uint4(0, 0, 0, 0);
    if (h0 && b < nrows && col < H)
      v = *reinterpret_cast<const uint4*>(h0 + (mb + b) * H + (col + u0) % H);
    *reinterpret_cast<uint4*>(hs + b * HP + col) = v;
  }
  if (tid == 0) *abort_flag = 0;
  float c[NT];
  {
    const bf16* s0 = GRU ? h0 : c0;
    bf16x8 cv = {};
    if (s0 && brow) cv = *reinterpret_cast<const bf16x8*>(s0 + (mb + fr) * H + ucol);
#pragma unroll
    for (int j = 0; j < NT; ++j) c[j] = lane_f<T>(cv, j);
  }
  float bn[NT];                                      // GRU: b_hh of gate n for the lane's units
#pragma unroll
  for (int j = 0; j < NT; ++j) bn[j] = 0.f;
  if constexpr (GRU) {
    if (p.bhn) {
      const f32x4* bp = reinterpret_cast<const f32x4*>(p.bhn + static_cast<int64_t>(mdl) * H + ucol);
      const f32x4 b0 = bp[0], b1 = bp[1];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bn[j] = b0[j];
        bn[4 + j] = b1[j];
      }
    }
  }
  const __amdgpu_buffer_rsrc_t ors = part_rsrc(static_cast<bf16*>(p.out) + mb * p.steps * H,
                                               static_cast<uint32_t>(nrows) * p.steps * H * 2);
  const __amdgpu_buffer_rsrc_t grs = part_rsrc(static_cast<const bf16*>(p.gx) + mb * p.steps * G,
                                               static_cast<uint32_t>(nrows) * p.steps * G * 2);
  const __amdgpu_buffer_rsrc_t xrs = part_rsrc(p.xch + static_cast<int64_t>(unit) * 2 * 16 * H, 2 * 16 * H * 4);
  const uint32_t lane_row = static_cast<uint32_t>(brow ? fr : 0) * p.steps;   // b * steps for this lane
  bf16x8 gxn[4];
  auto load_gx = [&](int t) {
    const uint32_t off = ((lane_row + t) * G + ucol) * 2;
#pragma unroll
    for (int q = 0; q < NG; ++q)
      gxn[q] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(grs, off + q * H * 2, 0, 0));
  };
  load_gx(0);
  int* my_sync = p.sync + static_cast<int64_t>(unit) * kSyncInts;
  const uint32_t base = static_cast<uint32_t>(sync_load(my_sync + kSyncBase));
  __syncthreads();

  // Are all parts of this model on one XCD?  Then exchange stores are plain: they write
  // through the CU's L1 into that XCD's L2, where the readers' device-scope (sc1) loads
  // find them (about 500 cycles store to load, measured); otherwise the stores are
  // device-scope as well, written through to the memory side that all XCDs share.  Each part publishes (tag of step 0, XCD + 1) and
  // reads the others' entries; every part reaches the same verdict.
  bool local = false;
  {
    const uint32_t tag0 = base & 0xFFFFu;
    if (tid == 0) {
      const uint32_t xcc = __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 0xFu;   // HW_REG_XCC_ID
      sync_store(my_sync + kSyncXcc + part, static_cast<int>((tag0 << 16) | (xcc + 1)));
    }
    if (w == 0) {
      uint32_t mine = 0, got = 0;
      bool ok = true;
      if (lane < P) {
        int spins = 0;
        while (true) {
          if (spins++ >= p.spin_limit) {
            ok = false;
            break;
          }
          got = static_cast<uint32_t>(sync_load(my_sync + kSyncXcc + lane));
          if ((got >> 16) == tag0 && (got & 0xFFFFu) != 0) break;
          __builtin_amdgcn_s_sleep(1);
        }
      }
      mine = __shfl(got, 0, 64);
      const bool same = __all(lane >= P || got == mine);
      if (lane == 0) xcd_flag[0] = same ? 1 : 0;
      if (!ok) *abort_flag = 1;
    }
    __syncthreads();
    local = xcd_flag[0] != 0;
  }

  bf16x8 hv = {};
  // LSTM exchange: h_t travels as its own 16-bit values, 8 to a 16-byte chunk.  |h| =
  // |o tanh(c)| <= 1, so bit 14 (the top exponent bit of bf16 and of fp16) is 0 in every h;
  // it carries the tag ((g >> 1) & 1) of global step g = base + t, and the slot is g & 1, so
  // a value left in the slot from step g - 2 always fails the check (the tag base is 16
  // bits wide, a multiple of the period 4).  A value from step g - 4 would pass: hence every
  // step is published, a launch's last one included, and a slot never holds one that old.
  // A NaN h (exponent bits all ones) travels as
  // the code 1.5, a value no h takes, which the reader turns back into NaN.  Chunk e of this
  // workgroup (8 values) is row e / CPR_H, slice r / 16 (skipping our own), units 8 (r % 16)
  // onward.
  constexpr uint32_t kTagBits = 0x40004000u;
  constexpr bool kF16 = std::is_same<T, f16>::value;
  constexpr uint32_t kHMax = kF16 ? 0x3C00u : 0x3F80u;      // |1.0|
  constexpr uint32_t kHNanCode = kF16 ? 0x3E00u : 0x3FC0u;  // 1.5
  constexpr uint32_t kHNan = kF16 ? 0x7E00u : 0x7FC0u;
  constexpr int CPR_H = (P - 1) * kPartUnits / 8;          // remote chunks per row
  constexpr int CPT_H = (16 * CPR_H + kPartThreads - 1) / kPartThreads;
  auto put_h = [&](auto pol, uint32_t g, bool nan_any) {
    constexpr int POL = decltype(pol)::value;
    u32x4 hw = __builtin_bit_cast(u32x4, hv);
    if (nan_any) {                                   // rare: a NaN h becomes the code
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        uint32_t lo = hw[k] & 0xFFFFu, hi = hw[k] >> 16;
        if ((lo & 0x7FFFu) > kHMax) lo = kHNanCode;
        if ((hi & 0x7FFFu) > kHMax) hi = kHNanCode;
        hw[k] = lo | (hi << 16);
      }
    }
    const uint32_t m = ((g >> 1) & 1u) ? kTagBits : 0u;
#pragma unroll
    for (int k = 0; k < 4; ++k) hw[k] |= m;
    const uint32_t xo = (((g & 1u) * 16 + fr) * H + ucol) * 2;
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, hw), xrs, xo, 0, POL);
  };
  auto chunk_h = [&](int k, int& b, int& col) {
    const int e = tid + k * kPartThreads;
    b = e / CPR_H;
    const int r = e - b * CPR_H;
    int q = r / (kPartUnits / 8);
    q += (q >= part) ? 1 : 0;
    col = q * kPartUnits + (r % (kPartUnits / 8)) * 8;
  };
  auto get_h = [&](uint32_t g, auto after) {
    const uint32_t slot = (g & 1u) * 16;
    const uint32_t want = ((g >> 1) & 1u) ? kTagBits : 0u;
    uint32_t pending = 0;
#pragma unroll
    for (int k = 0; k < CPT_H; ++k) {
      int b, col;
      chunk_h(k, b, col);
      if (b < nrows) pending |= 1u << k;
    }
    int spins = 0;
    bool after_done = false;
    while (pending) {
      if (spins++ >= p.spin_limit) {
        *abort_flag = 1;
        break;
      }
      asm volatile("" ::: "memory");                 // every round issues its loads anew
      u32x4 v[CPT_H];
#pragma unroll
      for (int k = 0; k < CPT_H; ++k) {
        int b, col;
        chunk_h(k, b, col);
        if (pending & (1u << k))
          v[k] = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, ((slot + b) * H + col) * 2, 0, kSc1));
      }
      if (!after_done) {
        after();
        after_done = true;
      }
#pragma unroll
      for (int k = 0; k < CPT_H; ++k) {
        if (!(pending & (1u << k))) continue;
        const uint32_t any = v[k][0] | v[k][1] | v[k][2] | v[k][3];
        const uint32_t all = v[k][0] & v[k][1] & v[k][2] & v[k][3];
        if (want ? (all & kTagBits) != kTagBits : (any & kTagBits) != 0u) continue;
        u32x4 hx;
#pragma unroll
        for (int q = 0; q < 4; ++q) hx[q] = v[k][q] & ~kTagBits;
        // the largest magnitude of the 8 values: above |1.0| only for the NaN code
        u16x2 mx = __builtin_bit_cast(u16x2, hx[0] & 0x7FFF7FFFu);
#pragma unroll
        for (int q = 1; q < 4; ++q) mx = __builtin_elementwise_max(mx, __builtin_bit_cast(u16x2, hx[q] & 0x7FFF7FFFu));
        if (mx[0] > kHMax || mx[1] > kHMax) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            uint32_t lo = hx[q] & 0xFFFFu, hi = hx[q] >> 16;
            if ((lo & 0x7FFFu) > kHMax) lo = kHNan;
            if ((hi & 0x7FFFu) > kHMax) hi = kHNan;
            hx[q] = lo | (hi << 16);
          }
        }
        int b, col;
        chunk_h(k, b, col);
        *reinterpret_cast<u32x4*>(hs + b * HP + (col - u0 + H) % H) = hx;
        pending &= ~(1u << k);
      }
      if (pending) __builtin_amdgcn_s_sleep(1);
    }
    if (!after_done) after();
  };
  // GRU exchange (its h may exceed 1 in magnitude when h0 does): one step's exchange with
  // cache policy POL: write the lane's 8 values of h_t, then
  // copy the other parts' slices of h_t (rows < batch) into LDS.  Chunk e of this
  // workgroup (16 bytes = 4 exchange words) is row e / CPR, slice r / 32 (skipping our
  // own), units 4 (r % 32) onward; a thread polls its chunks in groups of PG.
  auto put = [&](auto pol, int t, uint32_t tag) {
    constexpr int POL = decltype(pol)::value;
    const u32x4 hw = __builtin_bit_cast(u32x4, hv);   // bf16 pairs: (odd << 16) | even
    i32x4 lo, hi;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      lo[2 * k] = static_cast<int>((hw[k] << 16) | tag);
      lo[2 * k + 1] = static_cast<int>((hw[k] & 0xFFFF0000u) | tag);
      hi[2 * k] = static_cast<int>((hw[k + 2] << 16) | tag);
      hi[2 * k + 1] = static_cast<int>((hw[k + 2] & 0xFFFF0000u) | tag);
    }
    const uint32_t xo = (((t & 1) * 16 + fr) * H + ucol) * 4;
    __builtin_amdgcn_raw_buffer_store_b128(lo, xrs, xo, 0, POL);
    __builtin_amdgcn_raw_buffer_store_b128(hi, xrs, xo + 16, 0, POL);
  };
  auto chunk = [&](int k, int& b, int& col) {
    const int e = tid + k * kPartThreads;
    b = e / CPR;
    const int r = e - b * CPR;
    int q = r / (kPartUnits / 4);
    q += (q >= part) ? 1 : 0;
    col = q * kPartUnits + (r % (kPartUnits / 4)) * 4;
  };
  auto get = [&](int t, uint32_t tag, auto after) {
    constexpr int PG = CPT;
    bool after_done = false;
    const uint32_t slot = static_cast<uint32_t>(t & 1) * 16;
#pragma unroll
    for (int k0 = 0; k0 < CPT; k0 += PG) {
      uint32_t pending = 0;
#pragma unroll
      for (int k = 0; k < PG; ++k) {
        int b, col;
        chunk(k0 + k, b, col);
        if (k0 + k < CPT && b < nrows) pending |= 1u << k;
      }
      int spins = 0;
      while (pending) {
        if (spins++ >= p.spin_limit) {
          *abort_flag = 1;
          break;
        }
        asm volatile("" ::: "memory");   // every round issues its loads anew
        u32x4 v[PG];
#pragma unroll
        for (int k = 0; k < PG; ++k) {
          int b, col;
          chunk(k0 + k, b, col);
          if (pending & (1u << k))
            v[k] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, ((slot + b) * H + col) * 4, 0, kSc1));
        }
        if (!after_done) {
          after();
          after_done = true;
        }
#pragma unroll
        for (int k = 0; k < PG; ++k) {
          if (!(pending & (1u << k))) continue;
          if ((v[k][0] & 0xFFFFu) == tag && (v[k][1] & 0xFFFFu) == tag && (v[k][2] & 0xFFFFu) == tag &&
              (v[k][3] & 0xFFFFu) == tag) {
            int b, col;
            chunk(k0 + k, b, col);
            *reinterpret_cast<uint2*>(hs + b * HP + (col - u0 + H) % H) =
                make_uint2((v[k][0] >> 16) | (v[k][1] & 0xFFFF0000u), (v[k][2] >> 16) | (v[k][3] & 0xFFFF0000u));
            pending &= ~(1u << k);
          }
        }
        if (pending) __builtin_amdgcn_s_sleep(1);
      }
    }
    if (!after_done) after();
  };

  bool aborted = *abort_flag != 0;
  // LDS columns are rotated by this part's first unit (column c' holds h column c' + u0),
  // so this part's own k-steps are 0..KPP-1 and every read is the row base plus an
  // immediate offset.  The own k-steps of step t + 1 run while h_t is being exchanged.
  const bf16x8* wlw = wl + w * NF * 64 + lane;       // this lane's LDS fragments
  const bf16* hrow = hs + fr * HP + g * 8;           // this lane's h columns
  f32x4 acc[NT];
  // LSTM: the accumulators start from gates_x, which frees its registers a whole step
  // before the next cell update, so gates_x of step t + 1 is loaded at the top of step t,
  // ahead of every exchange load of the step (vmcnt retires loads in order: a load issued
  // behind the exchange polls would hold up every poll round after the first).  GRU keeps
  // gates_x apart from the hidden part of n, so it loads one step ahead in the exchange.
#pragma unroll
  for (int j = 0; j < NT; ++j) acc[j] = GRU ? f32x4{0.f, 0.f, 0.f, 0.f} : gx_acc<T>(gxn, j);
  mfma_steps<T, SL, NA, XL, KS, SH, 0, KPP, 0, NT>(acc, wa, wv, wlw, hrow);
  for (int t = 0; t < p.steps && !aborted; ++t) {
    if constexpr (!GRU) {
      if (t + 1 < p.steps) load_gx(t + 1);
    }
    // gate slots = h_{t-1} W_hh^T (MFMA; own columns already in acc), in two tile groups,
    // so that the cell update of the first group can run between the second group's MFMAs
    // (the h fragments are read once per group); gates_x (x W_ih^T + the folded biases) is
    // the LSTM's starting accumulator and joins the GRU's gates in the cell update
    mfma_steps<T, SL, NA, XL, KS, SH, KPP, KS, 0, NT / 2>(acc, wa, wv, wlw, hrow);
    mfma_steps<T, SL, NA, XL, KS, SH, KPP, KS, NT / 2, NT>(acc, wa, wv, wlw, hrow);
    // cell update of the lane's 8 units (hsum: NaN exactly when some h of the lane is)
    float hsum = 0.f;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      if constexpr (GRU) {
        // r, z, n in acc[j][0..2]; gates_x holds b_ir + b_hr, b_iz + b_hz and b_in; b_hn
        // joins the hidden part of n before r scales it (the torch.nn GRU cell)
        const float rg = sigmoid_f(acc[j][0] + lane_f<T>(gxn[0], j));
        const float zg = sigmoid_f(acc[j][1] + lane_f<T>(gxn[1], j));
        const float nn = tanh_f(lane_f<T>(gxn[2], j) + rg * (acc[j][2] + bn[j]));
        c[j] = (1.0f - zg) * nn + zg * c[j];
        set_lane<T>(hv, j, c[j]);
      } else {
        // i, f, g, o in acc[j][0..3], gates_x included
        const float ig = sigmoid_f(acc[j][0]);
        const float fg = sigmoid_f(acc[j][1]);
        const float gg = tanh_f(acc[j][2]);
        const float og = sigmoid_f(acc[j][3]);
        c[j] = fg * c[j] + ig * gg;
        const float h = og * tanh_f(c[j]);
        hsum += h;
        set_lane<T>(hv, j, h);
      }
    }
    const uint32_t tag = (base + static_cast<uint32_t>(t)) & 0xFFFFu;
    const bool more = t + 1 < p.steps;
    if constexpr (GRU) {
      if (brow && more) {
        if (local) put(std::integral_constant<int, 0>{}, t, tag);
        else put(std::integral_constant<int, kSc1>{}, t, tag);
      }
    } else if (brow) {
      // the last step is published too, although no part of this launch reads it: the
      // 1-bit tag repeats every 4 steps, so the next launch's step 1 (global step B + 1 with
      // B = base + steps) must find B - 1 in its slot, two steps old, not B - 3
      const bool nan_any = !(hsum == hsum);
      if (local) put_h(std::integral_constant<int, 0>{}, base + t, nan_any);
      else put_h(std::integral_constant<int, kSc1>{}, base + t, nan_any);
    }
    // the output row goes out after the exchange loads (GRU: behind the first poll round;
    // LSTM: once the exchange is complete): vmcnt counts stores and loads in order, so an
    // earlier store would hold up the exchange loads' waits
    auto put_out = [&]() {
      if (brow)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, hv), ors,
                                               ((lane_row + t) * H + ucol) * 2, 0, 0);
    };
    if (!more) {
      put_out();
      break;
    }
    lds_barrier();                                     // every wave has read h_{t-1}
    *reinterpret_cast<bf16x8*>(hs + fr * HP + (ucol - u0)) = hv;
    lds_barrier();                                     // this part's h_t is in LDS
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[j] = GRU ? f32x4{0.f, 0.f, 0.f, 0.f} : gx_acc<T>(gxn, j);
    mfma_steps<T, SL, NA, XL, KS, SH, 0, KPP, 0, NT>(acc, wa, wv, wlw, hrow);   // own columns of step t + 1
    // GRU: the output row and the next gates_x go out once the exchange loads are in flight:
    // the cell update of step t + 1 reads gates_x between that step's MFMAs, and a load
    // issued at the end of the step would still be on its way from HBM there
    auto out_and_gx = [&]() {
      put_out();
      load_gx(t + 1);
    };
    if constexpr (GRU) {
      get(t, tag, out_and_gx);
    } else {
      get_h(base + t, [] {});
      // every exchange load has been checked by now; an explicit vmcnt(0) tells the
      // compiler so (it counts the conditional poll loads as possibly in flight and would
      // otherwise wait for the next step's gates_x loads at the step's first LDS read)
      __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0) expcnt(7) lgkmcnt(15)
      put_out();
    }
    lds_barrier();
    aborted = *abort_flag != 0;
  }

  if (!aborted && brow) {
    const int64_t so = (mb + fr) * H + ucol;
    if (p.hn) *reinterpret_cast<bf16x8*>(static_cast<bf16*>(p.hn) + so) = hv;
    if (!GRU && p.cn) {
      bf16x8 cv;
#pragma unroll
      for (int j = 0; j < NT; ++j) set_lane<T>(cv, j, c[j]);
      *reinterpret_cast<bf16x8*>(static_cast<bf16*>(p.cn) + so) = cv;
    }
  }
  // the last part of the unit to finish advances the tag base for the next launch
  __syncthreads();
  if (tid == 0) {
    if (aborted) sync_store(p.status, 1);
    const int before = __hip_atomic_fetch_add(my_sync + kSyncDone, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (before == P - 1) {
      sync_store(my_sync + kSyncDone, 0);
      sync_store(my_sync + kSyncBase, static_cast<int>((base + static_cast<uint32_t>(p.steps)) & 0xFFFFu));
    }
  }
}

// counters, tag base and status zeroed; exchange slots filled with tag 0xFFFF; bias (fp32,
// [n, G]) = b_ih + b_hh, except that the GRU's gate n (columns >= fold of each model's G)
// takes b_ih alone and its b_hh goes to bhn (fp32, [n, H]); either bias may be null
template <typename T>
__global__ void part_prep_kernel(int* sync, int64_t nsync, uint32_t* xch, int64_t nxch, const T* b_ih,
                                 const T* b_hh, float* bias, int64_t nbias, int g, int fold, float* bhn,
                                 int hid) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < nsync) sync_store(sync + i, 0);
  if (i < nxch) __hip_atomic_store(xch + i, kTagFill, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (bias && i < nbias) {
    const int col = static_cast<int>(i % g);
    const float bh = b_hh ? to_f32(b_hh[i]) : 0.f;
    bias[i] = (b_ih ? to_f32(b_ih[i]) : 0.f) + (col < fold ? bh : 0.f);
    if (bhn && col >= fold) bhn[(i / g) * hid + (col - fold)] = bh;
  }
}

template <int H, typename T, int CELL>
bool part_kernel_fits() {
  const size_t lds = part_lds_bytes<H>();
  const void* fn = reinterpret_cast<const void*>(part_kernel<H, T, CELL>);
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) != hipSuccess)
    return false;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kPartThreads, lds) != hipSuccess) return false;
  return per_cu >= 1;
}

inline int64_t round256(int64_t v) { return (v + 255) & ~static_cast<int64_t>(255); }

inline int64_t part_gates(const wc_rnn_args* a) { return (a->cell == WC_CELL_GRU ? 3 : 4) * a->hidden; }
inline int64_t part_units(const wc_rnn_args* a) { return a->n * ((a->batch + 15) / 16); }

struct PartLayout {
  int64_t gx, bias, bhn, sync, xch, status, total;   // byte offsets into the workspace
};

PartLayout part_layout(const wc_rnn_args* a) {
  const int64_t g = part_gates(a), units = part_units(a);
  PartLayout l;
  l.gx = 0;
  l.bias = round256(a->n * a->batch * a->steps * g * 2);
  l.bhn = l.bias + round256(a->n * g * 4);
  l.xch = l.bhn + (a->cell == WC_CELL_GRU ? round256(a->n * a->hidden * 4) : 0);
  l.sync = l.xch + round256(units * 2 * 16 * a->hidden * 4);
  l.status = l.sync + round256(units * kSyncInts * 4);   // the counters and the status word are
  l.total = l.status + 256;                              // one contiguous int range
  return l;
}

template <int H, typename T, int CELL>
int32_t launch_part(const wc_rnn_args* a, hipStream_t st) {
  constexpr int P = H / kPartUnits;
  const PartLayout l = part_layout(a);
  char* ws = static_cast<char*>(a->workspace);
  PartParams p;
  p.n = static_cast<int>(a->n);
  p.rows = static_cast<int>(a->batch);
  p.chunks = (p.rows + 15) / 16;
  p.steps = static_cast<int>(a->steps);
  p.gx = ws + l.gx;
  p.w_hh = a->w_hh;
  p.h0 = a->h0;
  p.c0 = CELL == WC_CELL_LSTM ? a->c0 : nullptr;
  p.bhn = CELL == WC_CELL_GRU && a->b_hh ? reinterpret_cast<const float*>(ws + l.bhn) : nullptr;
  p.out = a->out;
  p.hn = a->h_n;
  p.cn = CELL == WC_CELL_LSTM ? a->c_n : nullptr;
  p.xch = reinterpret_cast<uint32_t*>(ws + l.xch);
  p.sync = reinterpret_cast<int*>(ws + l.sync);
  p.status = a->status ? static_cast<int*>(a->status) : reinterpret_cast<int*>(ws + l.status);
  p.spin_limit = g_spin_limit.load(std::memory_order_relaxed);
  const size_t lds = part_lds_bytes<H>();
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cap) != hipSuccess)
    return set_error(WC_ERR_ARG, "wc_rnn_recurrence: stream capture status unavailable");
  // WC_RNN_COOPERATIVE=0 makes the eager launch an ordinary one too, like the one under
  // capture (rocprofv3 7.2 crashes at exit after a cooperative launch and writes no trace)
  static const bool cooperative = [] {
    const char* v = getenv("WC_RNN_COOPERATIVE");
    return !(v && v[0] == '0' && v[1] == '\0');
  }();
  const void* fn = reinterpret_cast<const void*>(part_kernel<H, T, CELL>);
  // units of (model, 16-row chunk), at most one workgroup per compute unit per launch
  const int total = static_cast<int>(part_units(a));
  const int per_launch = device_cu_count() / P;
  for (int u = 0; u < total; u += per_launch) {
    const int units = total - u < per_launch ? total - u : per_launch;
    const int nwg = units * P;
    p.unit0 = u;
    p.remap = (nwg % 8 == 0 && (nwg / 8) % P == 0) ? 1 : 0;
    if (cap == hipStreamCaptureStatusNone && cooperative) {
      // co-residency of the whole grid is guaranteed, or the launch fails here
      void* args[] = {&p};
      const hipError_t e = hipLaunchCooperativeKernel(fn, dim3(nwg), dim3(kPartThreads), args,
                                                      static_cast<unsigned>(lds), st);
      if (e != hipSuccess)
        return set_error(static_cast<int32_t>(e), "wc_rnn_recurrence: cooperative launch of %d workgroups "
                         "failed: %s", nwg, hipGetErrorString(e));
    } else {
      // under graph capture (or WC_RNN_COOPERATIVE=0): an ordinary launch (part_plan checked
      // that one workgroup fits a compute unit, and no launch has more than the device's)
      part_kernel<H, T, CELL><<<dim3(nwg), dim3(kPartThreads), lds, st>>>(p);
      const int32_t rc = check_launch("wc_rnn_recurrence(partitioned)");
      if (rc) return rc;
    }
  }
  return WC_OK;
}

template <int H>
bool part_fits(const wc_rnn_args* a) {
  if (a->dtype == WC_F16)
    return a->cell == WC_CELL_GRU ? part_kernel_fits<H, f16, WC_CELL_GRU>() : part_kernel_fits<H, f16, WC_CELL_LSTM>();
  return a->cell == WC_CELL_GRU ? part_kernel_fits<H, bf16, WC_CELL_GRU>() : part_kernel_fits<H, bf16, WC_CELL_LSTM>();
}

template <int H>
int32_t part_dispatch(const wc_rnn_args* a, hipStream_t st) {
  if (a->dtype == WC_F16)
    return a->cell == WC_CELL_GRU ? launch_part<H, f16, WC_CELL_GRU>(a, st) : launch_part<H, f16, WC_CELL_LSTM>(a, st);
  return a->cell == WC_CELL_GRU ? launch_part<H, bf16, WC_CELL_GRU>(a, st) : launch_part<H, bf16, WC_CELL_LSTM>(a, st);
}

}  // namespace

bool part_plan(const wc_rnn_args* a) {
  if ((a->cell != WC_CELL_LSTM && a->cell != WC_CELL_GRU) || (a->dtype != WC_BF16 && a->dtype != WC_F16) ||
      a->batch < 1 || a->steps < 1 || a->steps > 0xFFFF)
    return false;
  if (a->hidden != 256 && a->hidden != 384 && a->hidden != 512) return false;
  const int64_t parts = a->hidden / kPartUnits;
  const int cus = device_cu_count();
  if (cus <= 0 || parts > cus) return false;
  // a unit's block of gates_x (16 rows) is addressed with 32-bit byte offsets
  if (16 * a->steps * part_gates(a) * 2 >= 0x7fffffffll) return false;
  for (const void* q : {a->w_hh, a->h0, a->c0, static_cast<const void*>(a->out),
                        static_cast<const void*>(a->h_n), static_cast<const void*>(a->c_n)})
    if (q && !aligned(q, 16)) return false;
  if (a->hidden == 256) return part_fits<256>(a);
  if (a->hidden == 384) return part_fits<384>(a);
  return part_fits<512>(a);
}

int64_t part_workspace_bytes(const wc_rnn_args* a) { return part_layout(a).total; }

int64_t part_status_offset(const wc_rnn_args* a) { return part_layout(a).status; }

int32_t part_set_spin_limit(int32_t polls) {
  return g_spin_limit.exchange(polls < 0 ? kSpinLimit : polls);
}

int32_t part_prepare(const wc_rnn_args* a, hipStream_t st, void** bias_f32) {
  const PartLayout l = part_layout(a);
  char* ws = static_cast<char*>(a->workspace);
  const int64_t g = part_gates(a);
  const int64_t nsync = (l.total - l.sync) / 4;
  const int64_t nxch = (l.sync - l.xch) / 4;
  const int64_t nbias = (a->b_ih || a->b_hh) ? a->n * g : 0;
  const bool gru = a->cell == WC_CELL_GRU;
  *bias_f32 = nbias ? ws + l.bias : nullptr;
  float* bhn = gru && a->b_hh ? reinterpret_cast<float*>(ws + l.bhn) : nullptr;
  const int fold = static_cast<int>(gru ? 2 * a->hidden : g);
  const int64_t items = std::max(std::max(nsync, nxch), nbias);
  const dim3 grid(static_cast<uint32_t>(cdiv(items, 256)));
  if (a->dtype == WC_F16)
    part_prep_kernel<f16><<<grid, 256, 0, st>>>(
        reinterpret_cast<int*>(ws + l.sync), nsync, reinterpret_cast<uint32_t*>(ws + l.xch), nxch,
        static_cast<const f16*>(a->b_ih), static_cast<const f16*>(a->b_hh), static_cast<float*>(*bias_f32), nbias,
        static_cast<int>(g), fold, bhn, static_cast<int>(a->hidden));
  else
    part_prep_kernel<bf16><<<grid, 256, 0, st>>>(
        reinterpret_cast<int*>(ws + l.sync), nsync, reinterpret_cast<uint32_t*>(ws + l.xch), nxch,
        static_cast<const bf16*>(a->b_ih), static_cast<const bf16*>(a->b_hh), static_cast<float*>(*bias_f32),
        nbias, static_cast<int>(g), fold, bhn, static_cast<int>(a->hidden));
  return check_launch("wc_rnn_input_projection(prep)");
}

int32_t part_recurrence(const wc_rnn_args* a, hipStream_t st) {
  if (a->hidden == 256) return part_dispatch<256>(a, st);
  if (a->hidden == 384) return part_dispatch<384>(a, st);
  return part_dispatch<512>(a, st);
}

}  // namespace wc
