// Internal interface shared by the recurrent kernels (rnn.hip) and the partitioned
// on-chip LSTM (rnn_part.hip).
#pragma once

#include "wc_common.h"

namespace wc {

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

// ---- partitioned on-chip LSTM (rnn_part.hip) ----
// true when the partitioned kernel runs these sizes on the current device
bool part_plan(const wc_rnn_args* a);
// workspace bytes and the byte offset of its status word under that plan
int64_t part_workspace_bytes(const wc_rnn_args* a);
int64_t part_status_offset(const wc_rnn_args* a);
// poll rounds after which a wait of launches made from now on gives up (0: at the first
// wait, < 0: the default); returns the previous value
int32_t part_set_spin_limit(int32_t polls);
// before the input projection: zero the plan's counters and status word, reset the
// exchange buffer, and write bias = b_ih + b_hh (fp32) into the workspace; *bias_f32
// receives its address (null when the layer has no bias)
int32_t part_prepare(const wc_rnn_args* a, hipStream_t st, void** bias_f32);
int32_t part_recurrence(const wc_rnn_args* a, hipStream_t st);

}  // namespace wc
