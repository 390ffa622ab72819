// Partitioned persistent LSTM recurrence (bf16; hidden 256, 384 or 512; batch <= 16).
//
// W_hh of one model (4H x H bf16: 2 MB at H = 512) exceeds one compute unit's
// registers and LDS, so P = H / 128 workgroups share a model, one per compute unit,
// for all T steps.  Workgroup `part` owns hidden units [128 part, 128 part + 128) and
// the 512 gate rows (i, f, g, o of each unit) of W_hh that feed them, held on-chip for
// the whole sequence: the first SL k-steps (32 columns each) in LDS, the next NA in
// AGPRs (loaded there directly and read in place as MFMA A operands), the rest in
// VGPRs.  This file is built with -amdgpu-mfma-vgpr-form so that accumulators live in
// VGPRs and the AGPR file is left to the weights.
//
// Per step a workgroup forms its gate pre-activations for all batch rows as MFMA tiles
// (A = W_hh rows, B = h_{t-1}^T read from LDS, C starts from gates_x), applies the
// cell update in registers (the fp32 cell state never leaves the chip), writes h_t to
// the output and to an exchange slot, and copies the other parts' slices of h_t from
// their exchange slots into its LDS.
//
// Lane layout (v_mfma_f32_16x16x32_bf16, wave w of 4, lane = 16 g + fr): row tile j
// (0..7) of wave w holds A row rho = gate (rho & 3) of unit 32 w + 8 (rho >> 2) + j,
// so the accumulator of lane (g, fr) holds all four gates of unit 32 w + 8 g + j for
// batch row fr.  A lane therefore owns 8 consecutive units of one batch row: its
// gates_x of a gate, its h_t and its cell state are 16-byte vectors, and the cell
// update needs no data exchange between lanes.
//
// Exchange.  Each exchanged value is one 32-bit word, (bf16 bits of h << 16) | tag,
// where tag = (base + t) mod 2^16 names the step; a reader polls the words it needs
// with device-scope (sc1) loads until every tag matches, so no separate flag, store
// fence or extra round trip is needed.  Writers use device-scope stores too, unless
// every part of the model runs on one XCD (read from HW_REG_XCC_ID at start), in which
// case plain stores into the shared L2 suffice and are faster.  There are
// two slots per model (step parity): a part cannot write step t + 2 into a slot before
// every other part has read step t from it, since it needs their step t + 1 first.
// `base` lives in the caller's workspace: the input projection zeroes it and fills
// the slots with tag 0xFFFF, and the last workgroup of a model to finish advances it
// by T, so a slot's stale tag is always 1 or 2 steps behind the one a reader expects.
// Every wait is bounded: past the limit (poll rounds, set by the host; 0 gives up
// at the first wait without polling) the workgroup records 1 in the status word
// and leaves (the outputs are then invalid).  The status word is the caller's own
// when one is passed (never cleared here), else a word of the workspace that the
// input projection zeroes.  The host launches the grid cooperatively, so all
// workgroups are co-resident or the launch fails.
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
constexpr uint32_t kTagFill = 0xFFFFu;

struct PartParams {
  int n, batch, steps, remap;
  int spin_limit;     // poll rounds of a wait before it gives up (0: at once)
  const bf16* gx;     // [n, batch, steps, 4H]: x W_ih^T + b_ih + b_hh, rounded to bf16
  const bf16* w_hh;   // [n, 4H, H]
  const bf16* h0;     // [n, batch, H] or null
  const bf16* c0;     // [n, batch, H] or null
  bf16* out;          // [n, batch, steps, H]
  bf16* hn;           // [n, batch, H] or null
  bf16* cn;           // [n, batch, H] or null
  uint32_t* xch;      // [n][2][16][H] exchange words
  int* sync;          // [n][kSyncInts]
  int* status;        // set to 1 when a wait gave up
};

std::atomic<int> g_spin_limit{kSpinLimit};

// Where the (k-step s, row tile j) fragments of W_hh live: s < SL in LDS, s < SL + NA in
// AGPRs, tiles j < XL of k-step SL + NA in LDS as well, the rest in VGPRs.
template <int H> struct PartCfg;
template <> struct PartCfg<256> { static constexpr int SL = 0, NA = 6, XL = 0; };
template <> struct PartCfg<384> { static constexpr int SL = 1, NA = 8, XL = 0; };
template <> struct PartCfg<512> { static constexpr int SL = 4, NA = 8, XL = 3; };

// The order in which the k-steps B..E-1 are visited: LDS-fed k-steps (s < SL, and SL + NA
// when XL > 0) alternate with register-fed ones, so the fragments of the next LDS-fed
// k-step are read while the MFMAs of a register-fed k-step run.
template <int SL, int NA, int XL, int B, int E>
struct KOrder {
  int s[E - B];
  bool lds[E - B];
  constexpr KOrder() : s(), lds() {
    int ls[E - B] = {}, rs[E - B] = {};
    int nl = 0, nr = 0;
    for (int k = B; k < E; ++k) {
      if (k < SL || (XL > 0 && k == SL + NA)) ls[nl++] = k;
      else rs[nr++] = k;
    }
    int o = 0, il = 0, ir = 0;
    while (il < nl || ir < nr) {
      if (il < nl) { s[o] = ls[il++]; lds[o++] = true; }
      if (ir < nr) { s[o] = rs[ir++]; lds[o++] = false; }
    }
  }
};

// acc[j] += the k-steps B..E-1 of (W_hh rows of tile j) x h^T for the tiles J0 <= j < J1:
// A fragments from LDS (wlw, this lane's fragment base), AGPRs (wa) or VGPRs (wv); B fragments
// from this lane's h row in LDS (hrow, k-step s at hrow + 32 s).
template <int SL, int NA, int XL, int B, int E, int J0, int J1, int NT, int RA, int RV>
__device__ __forceinline__ void mfma_steps(f32x4 (&acc)[NT], const bf16x8 (&wa)[RA][NT],
                                           const bf16x8 (&wv)[RV][NT], const bf16x8* wlw, const bf16* hrow) {
  static_assert(0 <= J0 && J0 < J1 && J1 <= NT, "tile range");
  constexpr KOrder<SL, NA, XL, B, E> ord;
  constexpr int N = E - B;
  bf16x8 lf[NT];                                     // LDS-fed fragments of the current / next k-step
  auto in_lds = [](int s, int j) { return s < SL || (XL > 0 && s == SL + NA && j < XL); };
  auto load_tile = [&](int s, int j) {
    if (s < SL) lf[j] = wlw[(s * NT + j) * 64];
    else if (in_lds(s, j)) lf[j] = wlw[(SL * NT + j) * 64];
  };
  bf16x8 hb = *reinterpret_cast<const bf16x8*>(hrow + ord.s[0] * 32);
  if (ord.lds[0]) {
#pragma unroll
    for (int j = J0; j < J1; ++j) load_tile(ord.s[0], j);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int s = ord.s[i];
    const bool nxt_lds = i + 1 < N && ord.lds[i + 1];
    const bf16x8 hc = hb;
    if (i + 1 < N) hb = *reinterpret_cast<const bf16x8*>(hrow + ord.s[i + 1] * 32);
    // a register-fed k-step: read all of the next LDS-fed k-step's fragments under its MFMAs
    if (!ord.lds[i] && nxt_lds) {
#pragma unroll
      for (int j = J0; j < J1; ++j) load_tile(ord.s[i + 1], j);
    }
#pragma unroll
    for (int j = J0; j < J1; ++j) {
      bf16x8 a;
      if (in_lds(s, j)) a = lf[j];
      else if (s < SL + NA) a = wa[s < SL + NA ? s - SL : 0][j];
      else a = wv[s < SL + NA ? 0 : s - SL - NA][j];
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, hc, acc[j], 0, 0, 0);
      // two LDS-fed k-steps in a row: refill tile j once its MFMA has taken it
      if (ord.lds[i] && nxt_lds) load_tile(ord.s[i + 1], j);
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

template <int H>
__global__ __launch_bounds__(kPartThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void lstm_part_kernel(PartParams p) {
  constexpr int NT = 8, KS = H / 32, P = H / kPartUnits;
  constexpr int SL = PartCfg<H>::SL, NA = PartCfg<H>::NA, XL = PartCfg<H>::XL, NV = KS - SL - NA;
  static_assert(NV >= 0 && P >= 2, "partition");
  constexpr int HP = H + 8;                          // LDS pitch of an h row (elements)
  constexpr int G = 4 * H;
  constexpr int KPP = kPartUnits / 32;               // k-steps of one part's columns
  constexpr int CPR = (P - 1) * kPartUnits / 4;      // remote 16-byte exchange chunks per row
  constexpr int CPT = (16 * CPR + kPartThreads - 1) / kPartThreads;
  extern __shared__ __attribute__((aligned(16))) char part_smem[];
  // LDS-resident W_hh fragments, [wave][f][64 lanes] x 16 bytes, f = 8 s + j for s < SL and
  // 8 SL + j for the XL tiles of k-step SL + NA: one wave's fragments lie within 64 KB of
  // its base, so every read is the base plus an immediate offset
  constexpr int NF = SL * NT + XL;
  bf16x8* wl = reinterpret_cast<bf16x8*>(part_smem);
  bf16* hs = reinterpret_cast<bf16*>(part_smem + (SL * NT + XL) * 4 * 1024);  // [16][HP] h_{t-1}
  int* abort_flag = reinterpret_cast<int*>(hs + 16 * HP);
  int* xcd_flag = abort_flag + 1;

  const int nwg = p.n * P;
  int id = blockIdx.x;
  if (p.remap) id = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);   // a model's parts share an XCD
  const int mdl = id / P, part = id - mdl * P;
  const int u0 = part * kPartUnits;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, g = lane >> 4, fr = lane & 15;
  const int ucol = u0 + w * 32 + g * 8;              // first of the lane's 8 units (model column)
  const bool brow = fr < p.batch;
  const int64_t mb = static_cast<int64_t>(mdl) * p.batch;

  // ---- W_hh rows of this part in LDS, AGPRs and VGPRs, loaded once ----
  bf16x8 wa[NA > 0 ? NA : 1][NT];
  bf16x8 wv[NV > 0 ? NV : 1][NT];
  {
    const bf16* wb = p.w_hh + static_cast<int64_t>(mdl) * G * H;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const bf16* row = wb + static_cast<int64_t>((fr & 3) * H + u0 + w * 32 + (fr >> 2) * 8 + j) * H + g * 8;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const bf16* src = row + ((s + part * KPP) % KS) * 32;   // rotated k-step s
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
  // ---- h_{-1} into LDS (rows >= batch stay zero), c_{-1} and gates_x of step 0 in registers ----
  for (int e = tid; e < 16 * (HP / 8); e += kPartThreads) {
    const int b = e / (HP / 8), col = (e - b * (HP / 8)) * 8;   // LDS column (rotated)
    uint4 v = make_uint4(0, 0, 0, 0);
    if (p.h0 && b < p.batch && col < H)
      v = *reinterpret_cast<const uint4*>(p.h0 + (mb + b) * H + (col + u0) % H);
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
  const __amdgpu_buffer_rsrc_t ors =
      part_rsrc(p.out + mb * p.steps * H, static_cast<uint32_t>(p.batch) * p.steps * H * 2);
  const __amdgpu_buffer_rsrc_t grs =
      part_rsrc(p.gx + mb * p.steps * G, static_cast<uint32_t>(p.batch) * p.steps * G * 2);
  const __amdgpu_buffer_rsrc_t xrs = part_rsrc(p.xch + static_cast<int64_t>(mdl) * 2 * 16 * H, 2 * 16 * H * 4);
  const uint32_t lane_row = static_cast<uint32_t>(brow ? fr : 0) * p.steps;   // b * steps for this lane
  bf16x8 gxn[4];
  auto load_gx = [&](int t) {
    const uint32_t off = ((lane_row + t) * G + ucol) * 2;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      gxn[q] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(grs, off + q * H * 2, 0, 0));
  };
  load_gx(0);
  int* my_sync = p.sync + static_cast<int64_t>(mdl) * kSyncInts;
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
  // One step's exchange with cache policy POL: write the lane's 8 values of h_t, then
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
  auto get = [&](int t, uint32_t tag) {
    constexpr int PG = CPT;
    const uint32_t slot = static_cast<uint32_t>(t & 1) * 16;
#pragma unroll
    for (int k0 = 0; k0 < CPT; k0 += PG) {
      uint32_t pending = 0;
#pragma unroll
      for (int k = 0; k < PG; ++k) {
        int b, col;
        chunk(k0 + k, b, col);
        if (k0 + k < CPT && b < p.batch) pending |= 1u << k;
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
  };

  bool aborted = *abort_flag != 0;
  // LDS columns are rotated by this part's first unit (column c' holds h column c' + u0),
  // so this part's own k-steps are 0..KPP-1 and every read is the row base plus an
  // immediate offset.  The own k-steps of step t + 1 run while h_t is being exchanged.
  const bf16x8* wlw = wl + w * NF * 64 + lane;       // this lane's LDS fragments
  const bf16* hrow = hs + fr * HP + g * 8;           // this lane's h columns
  f32x4 acc[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  mfma_steps<SL, NA, XL, 0, KPP, 0, NT>(acc, wa, wv, wlw, hrow);
  for (int t = 0; t < p.steps && !aborted; ++t) {
    // gates = h_{t-1} W_hh^T (MFMA; own columns already in acc) + gates_x (x W_ih^T + b_ih
    // + b_hh, added in the cell update)
    // in two tile groups, so that the cell update of the first group can run between the
    // second group's MFMAs (the h fragments are read once per group)
    mfma_steps<SL, NA, XL, KPP, KS, 0, NT / 2>(acc, wa, wv, wlw, hrow);
    mfma_steps<SL, NA, XL, KPP, KS, NT / 2, NT>(acc, wa, wv, wlw, hrow);
    // cell update of the lane's 8 units (i, f, g, o in acc[j][0..3])
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const float ig = sigmoid_f(acc[j][0] + static_cast<float>(gxn[0][j]));
      const float fg = sigmoid_f(acc[j][1] + static_cast<float>(gxn[1][j]));
      const float gg = tanh_f(acc[j][2] + static_cast<float>(gxn[2][j]));
      const float og = sigmoid_f(acc[j][3] + static_cast<float>(gxn[3][j]));
      c[j] = fg * c[j] + ig * gg;
      hv[j] = static_cast<bf16>(og * tanh_f(c[j]));
    }
    const uint32_t tag = (base + static_cast<uint32_t>(t)) & 0xFFFFu;
    const bool more = t + 1 < p.steps;
    if (brow && more) {
      if (local) put(std::integral_constant<int, 0>{}, t, tag);
      else put(std::integral_constant<int, kSc1>{}, t, tag);
    }
    // the output row goes out after the exchange: vmcnt counts stores and loads in
    // order, so an earlier store would hold up the exchange loads' wait
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
    for (int j = 0; j < NT; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    mfma_steps<SL, NA, XL, 0, KPP, 0, NT>(acc, wa, wv, wlw, hrow);   // own columns of step t + 1
    get(t, tag);
    put_out();
    load_gx(t + 1);                                    // lands during the next step's MFMAs
    lds_barrier();
    aborted = *abort_flag != 0;
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
  // the last part of the model to finish advances the tag base for the next launch
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

// counters, tag base and status zeroed; exchange slots filled with tag 0xFFFF;
// bias = b_ih + b_hh in fp32 (either may be null)
__global__ void part_prep_kernel(int* sync, int64_t nsync, uint32_t* xch, int64_t nxch, const bf16* b_ih,
                                 const bf16* b_hh, float* bias, int64_t nbias) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < nsync) sync_store(sync + i, 0);
  if (i < nxch) __hip_atomic_store(xch + i, kTagFill, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (bias && i < nbias)
    bias[i] = (b_ih ? static_cast<float>(b_ih[i]) : 0.f) + (b_hh ? static_cast<float>(b_hh[i]) : 0.f);
}

template <int H>
bool part_kernel_fits() {
  const size_t lds = part_lds_bytes<H>();
  const void* fn = reinterpret_cast<const void*>(lstm_part_kernel<H>);
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) != hipSuccess)
    return false;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kPartThreads, lds) != hipSuccess) return false;
  return per_cu >= 1;
}

inline int64_t round256(int64_t v) { return (v + 255) & ~static_cast<int64_t>(255); }

struct PartLayout {
  int64_t gx, bias, sync, xch, status, total;   // byte offsets into the workspace
};

PartLayout part_layout(const wc_rnn_args* a) {
  const int64_t g = 4 * a->hidden;
  PartLayout l;
  l.gx = 0;
  l.bias = round256(a->n * a->batch * a->steps * g * 2);
  l.xch = l.bias + round256(a->n * g * 4);
  l.sync = l.xch + round256(a->n * 2 * 16 * a->hidden * 4);
  l.status = l.sync + round256(a->n * kSyncInts * 4);   // the counters and the status word are
  l.total = l.status + 256;                             // one contiguous int range
  return l;
}

template <int H>
int32_t launch_part(const wc_rnn_args* a, hipStream_t st) {
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
  if (cap == hipStreamCaptureStatusNone && cooperative) {
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
  // under graph capture (or WC_RNN_COOPERATIVE=0): an ordinary launch (part_plan checked
  // that the grid fits the device one workgroup per compute unit)
  lstm_part_kernel<H><<<dim3(nwg), dim3(kPartThreads), lds, st>>>(p);
  return check_launch("wc_rnn_recurrence(partitioned)");
}

}  // namespace

bool part_plan(const wc_rnn_args* a) {
  if (a->cell != WC_CELL_LSTM || a->dtype != WC_BF16 || a->batch < 1 || a->batch > 16 || a->steps < 1 ||
      a->steps > 0xFFFF)
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
  if (a->hidden == 256) return part_kernel_fits<256>();
  if (a->hidden == 384) return part_kernel_fits<384>();
  return part_kernel_fits<512>();
}

int64_t part_workspace_bytes(const wc_rnn_args* a) { return part_layout(a).total; }

int64_t part_status_offset(const wc_rnn_args* a) { return part_layout(a).status; }

int32_t part_set_spin_limit(int32_t polls) {
  return g_spin_limit.exchange(polls < 0 ? kSpinLimit : polls);
}

int32_t part_prepare(const wc_rnn_args* a, hipStream_t st, void** bias_f32) {
  const PartLayout l = part_layout(a);
  char* ws = static_cast<char*>(a->workspace);
  const int64_t g = 4 * a->hidden;
  const int64_t nsync = (l.total - l.sync) / 4;
  const int64_t nxch = (l.sync - l.xch) / 4;
  const int64_t nbias = (a->b_ih || a->b_hh) ? a->n * g : 0;
  *bias_f32 = nbias ? ws + l.bias : nullptr;
  const int64_t items = std::max(std::max(nsync, nxch), nbias);
  part_prep_kernel<<<static_cast<uint32_t>(cdiv(items, 256)), 256, 0, st>>>(
      reinterpret_cast<int*>(ws + l.sync), nsync, reinterpret_cast<uint32_t*>(ws + l.xch), nxch,
      static_cast<const bf16*>(a->b_ih), static_cast<const bf16*>(a->b_hh), static_cast<float*>(*bias_f32), nbias);
  return check_launch("wc_rnn_input_projection(prep)");
}

int32_t part_recurrence(const wc_rnn_args* a, hipStream_t st) {
  if (a->hidden == 256) return launch_part<256>(a, st);
  if (a->hidden == 384) return launch_part<384>(a, st);
  return launch_part<512>(a, st);
}

}  // namespace wc
