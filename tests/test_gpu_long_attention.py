"""Long sequences through WideAttention (GPU): beyond the fused kernel's S <= 512, the flash-style
general kernel streams K/V tiles through LDS with an online softmax.  Reference: for every model,
its nn.MultiheadAttention in fp64 on the GPU (wide_attention.py:178-238 restates exactly that
stack per model).  Bars: fp32 1e-5, bf16 2e-2 (normwise)."""

import pytest
import torch
import torch.nn as nn

from tests._util import rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
BAR = {torch.float32: 1e-5, torch.bfloat16: 2e-2}


def _mods(n, d, h, seed):
    torch.manual_seed(seed)
    mods = [nn.MultiheadAttention(d, h, batch_first=True) for _ in range(n)]
    with torch.no_grad():
        for m in mods:
            m.in_proj_bias.uniform_(-0.1, 0.1)
            m.out_proj.bias.uniform_(-0.1, 0.1)
    return mods


@pytest.mark.parametrize("n,b,s,d,h,dtype,causal", [
    (2, 1, 4096, 256, 2, torch.bfloat16, False),       # head dim 128
    (2, 1, 4096, 256, 2, torch.bfloat16, True),
    (2, 2, 2048, 128, 2, torch.float32, False),        # head dim 64
    (1, 1, 2048, 128, 2, torch.float32, True),
    (2, 1, 1031, 64, 2, torch.bfloat16, True),         # head dim 32, a ragged last key tile
])
def test_long_self_attention(hip, n, b, s, d, h, dtype, causal):
    import wide_compiler as wc
    mods = _mods(n, d, h, s + d)
    wide = wc.WideAttention.from_modules(mods).to(DEV, dtype).eval()
    x = torch.randn(n, b, s, d, device=DEV).to(dtype)
    mask = torch.triu(torch.full((s, s), float("-inf"), device=DEV, dtype=torch.float64), 1) if causal else None
    with torch.no_grad():
        y = wide(x, is_causal=causal)
        ref = torch.stack([m.to(DEV).double()(x[q].double(), x[q].double(), x[q].double(), need_weights=False,
                                               attn_mask=mask)[0] for q, m in enumerate(mods)])
    assert rel_err(y, ref) <= BAR[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_long_cross_attention(hip, dtype):
    """37 queries over 4096 keys (MHA mode: separate key and value inputs)."""
    import wide_compiler as wc
    n, b, tq, tkv, d, h = 2, 2, 37, 4096, 128, 2
    mods = _mods(n, d, h, 77)
    wide = wc.WideAttention.from_modules(mods).to(DEV, dtype).eval()
    q_in, k_in, v_in = (torch.randn(n, b, t, d, device=DEV).to(dtype) for t in (tq, tkv, tkv))
    with torch.no_grad():
        y, _ = wide(q_in, k_in, v_in)
        ref = torch.stack([m.to(DEV).double()(q_in[i].double(), k_in[i].double(), v_in[i].double(),
                                               need_weights=False)[0] for i, m in enumerate(mods)])
    assert rel_err(y, ref) <= BAR[dtype]


@pytest.mark.parametrize("dh", [1, 8, 20, 24, 40, 48, 72, 80, 96, 112, 160, 200, 256])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("mode", ["plain", "causal", "mask", "cross"])
def test_any_head_dim(hip, dh, dtype, mode):
    """Head dims outside the vector kernel's 16 / 32 / 64 / 128 (scaled_dot_product_attention takes
    any, and the reference passes every head dim to it, wide_attention.py:212-231): the general
    form pads the scores' head dim and splits output columns past 128 into launches.  fp32 stops
    at 128 (its 256-wide K tiles would not fit in LDS) and says so."""
    import wide_compiler as wc
    from wide_compiler import _hip
    heads = 3 if dh <= 128 else 2
    d = heads * dh
    n, b, sq = 2, 2, 70
    skv = 45 if mode == "cross" else sq
    mods = _mods(n, d, heads, dh)
    wide = wc.WideAttention.from_modules(mods).to(DEV, dtype).eval()
    q_in = torch.randn(n, b, sq, d, device=DEV).to(dtype)
    k_in = torch.randn(n, b, skv, d, device=DEV).to(dtype) if mode == "cross" else q_in
    v_in = torch.randn(n, b, skv, d, device=DEV).to(dtype) if mode == "cross" else q_in
    mask = (torch.randn(sq, skv, device=DEV) * 2) if mode == "mask" else None
    if dtype == torch.float32 and dh > 128:
        with pytest.raises(_hip.WideKernelError, match="head dim"):
            with torch.no_grad():
                wide(q_in, is_causal=mode == "causal", attn_mask=mask)
        return
    with torch.no_grad():
        if mode == "cross":
            y, _ = wide(q_in, k_in, v_in)
        else:
            y = wide(q_in, is_causal=mode == "causal", attn_mask=mask)
        ref_mask = None
        if mode == "causal":
            ref_mask = torch.triu(torch.full((sq, sq), float("-inf"), device=DEV, dtype=torch.float64), 1)
        elif mode == "mask":
            ref_mask = mask.double()
        ref = torch.stack([m.to(DEV).double()(q_in[i].double(), k_in[i].double(), v_in[i].double(),
                                               need_weights=False, attn_mask=ref_mask)[0]
                           for i, m in enumerate(mods)])
    bar = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-3}[dtype]
    assert rel_err(y, ref) <= bar
