"""
CPU restatement of the reference wide primitives (test infrastructure only).

Every function follows one reference function op-for-op -- same torch ops, same order,
same dtype flow -- so that for bf16 inputs the rounding points are the reference's.
Functions take plain tensors (the reference's parameter layouts) and run on the CPU.

Pins (tests/test_oracle.py): each function is checked against an independent
implementation -- the per-model torch.nn modules the reference validates against
(benchmark_schema.py:108-152, wide_gru.py:453-488), float64 brute force on tiny shapes,
and closed forms -- with inputs chosen so a dropped term, swapped gate, wrong sign or
transposed operand fails.
"""

from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F
from torch import Tensor


# ---------------------------------------------------------------------------------------
# boundary (ensemble_util.py, traced_wide.py)
# ---------------------------------------------------------------------------------------

def pack_inputs(inputs: Sequence[Tensor]) -> Tensor:
    """ensemble_util.py:41-60."""
    if not inputs:
        raise ValueError("inputs list is empty")
    stacked = torch.stack(list(inputs), dim=1)
    b, n = stacked.shape[0], stacked.shape[1]
    rest = stacked.shape[2:]
    if len(rest) == 0:
        return stacked.view(b, n)
    return stacked.view(b, n * rest[0], *rest[1:])


def unpack_outputs(output: Tensor, n: int) -> List[Tensor]:
    """ensemble_util.py:83-101."""
    b = output.shape[0]
    nf = output.shape[1]
    if nf % n != 0:
        raise ValueError(f"Cannot split dim 1 ({nf}) into {n} equal parts")
    r = output.view(b, n, nf // n, *output.shape[2:])
    return [r[:, i] for i in range(n)]


def to_nfirst(x: Tensor, n: int) -> Tensor:
    """traced_wide.py:463-469."""
    b, nc = x.shape[0], x.shape[1]
    return x.view(b, n, nc // n, *x.shape[2:]).movedim(1, 0)


def to_packed(out: Tensor) -> Tensor:
    """traced_wide.py:524-532."""
    if isinstance(out, tuple):
        out = out[0]
    n, b, c = out.shape[0], out.shape[1], out.shape[2]
    return out.movedim(0, 1).reshape(b, n * c, *out.shape[3:])


# ---------------------------------------------------------------------------------------
# primitives
# ---------------------------------------------------------------------------------------

def linear(x: Tensor, weight: Tensor, bias: Optional[Tensor]) -> Tensor:
    """WideLinear._forward_einsum, wide_linear.py:157-173."""
    n, o, i = weight.shape
    batch = x.shape[1:-1]
    x = x.reshape(n, -1, i)
    out = torch.einsum("noi,nbi->nbo", weight, x)
    if bias is not None:
        out = out + bias.unsqueeze(1)
    return out.reshape(n, *batch, o)


def conv2d(x: Tensor, weight: Tensor, bias: Optional[Tensor], n: int, stride=(1, 1), padding=(0, 0),
           dilation=(1, 1)) -> Tensor:
    """WideConv2d.forward (grouped strategy), wide_conv2d.py:176-194; weight [N*Co, Ci, kh, kw]."""
    nn_, b, c, h, w = x.shape
    xp = x.permute(1, 0, 2, 3, 4).reshape(b, n * c, h, w)
    out = F.conv2d(xp, weight, bias, stride=stride, padding=padding, dilation=dilation, groups=n)
    b, nco, ho, wo = out.shape
    return out.view(b, n, nco // n, ho, wo).permute(1, 0, 2, 3, 4).contiguous()


def conv3d(x: Tensor, weight: Tensor, bias: Optional[Tensor], n: int, stride=(1, 1, 1), padding=(0, 0, 0),
           dilation=(1, 1, 1)) -> Tensor:
    """WideConv3d.forward (grouped strategy), wide_conv3d.py:102-124; weight [N*Co, Ci, kd, kh, kw]."""
    nn_, b, c, d, h, w = x.shape
    xp = x.permute(1, 0, 2, 3, 4, 5).reshape(b, n * c, d, h, w)
    out = F.conv3d(xp, weight, bias, stride=stride, padding=padding, dilation=dilation, groups=n)
    b, nco, do, ho, wo = out.shape
    return out.view(b, n, nco // n, do, ho, wo).permute(1, 0, 2, 3, 4, 5).contiguous()


def conv1d(x: Tensor, weight: Tensor, bias: Optional[Tensor], n: int, stride: int = 1, padding: int = 0,
           dilation: int = 1) -> Tensor:
    """WideConv1d.forward (grouped strategy), wide_conv1d.py:125-141; weight [N*Co, Ci, k]."""
    nn_, b, c, l = x.shape
    xp = x.permute(1, 0, 2, 3).reshape(b, n * c, l)
    out = F.conv1d(xp, weight, bias, stride=stride, padding=padding, dilation=dilation, groups=n)
    b, nco, lo = out.shape
    return out.view(b, n, nco // n, lo).permute(1, 0, 2, 3).contiguous()


def batchnorm_eval(x: Tensor, weight: Optional[Tensor], bias: Optional[Tensor], running_mean: Tensor,
                   running_var: Tensor, eps: float, n: int) -> Tensor:
    """WideBatchNorm2d.forward in eval mode, wide_batchnorm_2d.py:60-71 (also BatchNorm1d's)."""
    shape = x.shape
    b, c = shape[1], shape[2]
    perm = [1, 0] + list(range(2, x.dim()))
    xp = x.permute(*perm).reshape(b, n * c, *shape[3:])
    out = F.batch_norm(xp, running_mean, running_var, weight, bias, training=False, momentum=0.0, eps=eps)
    return out.view(b, n, c, *shape[3:]).permute(*perm).contiguous()


def layernorm(x: Tensor, weight_flat: Tensor, bias_flat: Tensor, n: int, eps: float) -> Tensor:
    """WideLayerNorm.forward, wide_layernorm.py:48-67 (manual mean / biased var)."""
    d = x.shape[-1]
    weight = weight_flat.view(n, d)
    bias = bias_flat.view(n, d)
    for _ in range(x.dim() - 2):
        weight = weight.unsqueeze(1)
        bias = bias.unsqueeze(1)
    mean = x.mean(dim=-1, keepdim=True)
    var = x.var(dim=-1, unbiased=False, keepdim=True)
    x = (x - mean) / torch.sqrt(var + eps)
    return x * weight + bias


def group_norm(x: Tensor, weight: Optional[Tensor], bias: Optional[Tensor], groups: int, eps: float) -> Tensor:
    """WideGroupNorm.forward (fused strategy), wide_groupnorm.py:89-117: nn.GroupNorm(N*G, N*C) over the
    channel-packed view.  x [N, B, C, *spatial]; each (model, batch row, group) is normalised over its
    C/G channels x spatial with the biased variance; weight / bias [N*C] (model i's channel c at i*C + c)
    or None."""
    n, b, c = x.shape[:3]
    xg = x.reshape(n, b, groups, -1)
    mean = xg.mean(dim=-1, keepdim=True)
    var = xg.var(dim=-1, unbiased=False, keepdim=True)
    y = ((xg - mean) / torch.sqrt(var + eps)).reshape(x.shape)
    if weight is not None:
        shape = (n, 1, c) + (1,) * (x.dim() - 3)
        y = y * weight.reshape(shape) + bias.reshape(shape)
    return y


def instance_norm(x: Tensor, weight: Optional[Tensor], bias: Optional[Tensor], eps: float,
                  running_mean: Optional[Tensor] = None, running_var: Optional[Tensor] = None) -> Tensor:
    """WideInstanceNorm1d/2d.forward (fused strategy), wide_instancenorm.py:82-101 / 213-232:
    nn.InstanceNorm*(N*C) on the channel-packed view -- instance statistics per (model, batch row,
    channel), or, in eval mode with track_running_stats, the running statistics."""
    if running_mean is not None:
        return batchnorm_eval(x, weight, bias, running_mean, running_var, eps, x.shape[0])
    return group_norm(x, weight, bias, x.shape[2], eps)


def embedding(weight: Tensor, ids: Tensor) -> Tensor:
    """WideEmbedding._forward_indexed, wide_embedding.py:100-102 (shared ids)."""
    return weight[:, ids]


def embedding_per_model(weight: Tensor, ids: Tensor) -> Tensor:
    """Model i looks up its own ids[i]: the sequential strategy's F.embedding (wide_embedding.py:130)
    applied per model to that model's ids."""
    return torch.stack([F.embedding(ids[i], weight[i]) for i in range(weight.shape[0])], dim=0)


def gru(x: Tensor, weight_ih: Tensor, weight_hh: Tensor, bias_ih: Optional[Tensor],
        bias_hh: Optional[Tensor], h_0: Optional[Tensor] = None) -> Tuple[Tensor, Tensor]:
    """WideGRU._forward_fused, wide_gru.py:159-213."""
    n = weight_ih.shape[0]
    h = weight_hh.shape[2]
    _, b, t, _ = x.shape
    gates_x = torch.einsum("nbti,ngi->nbtg", x, weight_ih)
    if bias_ih is not None:
        gates_x = gates_x + bias_ih.view(n, 1, 1, 3 * h)
    hs = h_0.contiguous() if h_0 is not None else torch.zeros(n, b, h, device=x.device, dtype=x.dtype)
    outs = []
    for step in range(t):
        gates_h = torch.einsum("nbh,ngh->nbg", hs, weight_hh)
        if bias_hh is not None:
            gates_h = gates_h + bias_hh.view(n, 1, 3 * h)
        gx = gates_x[:, :, step]
        gx_r, gx_z, gx_n = gx.chunk(3, dim=-1)
        gh_r, gh_z, gh_n = gates_h.chunk(3, dim=-1)
        r = torch.sigmoid(gx_r + gh_r)
        z = torch.sigmoid(gx_z + gh_z)
        nn_ = torch.tanh(gx_n + r * gh_n)
        hs = (1 - z) * nn_ + z * hs
        outs.append(hs)
    return torch.stack(outs, dim=2), hs


def lstm(x: Tensor, weight_ih: Tensor, weight_hh: Tensor, bias_ih: Optional[Tensor],
         bias_hh: Optional[Tensor], hx: Optional[Tuple[Tensor, Tensor]] = None
         ) -> Tuple[Tensor, Tuple[Tensor, Tensor]]:
    """WideLSTM._forward_fused, wide_lstm.py:169-234, on the diagonal blocks
    (weight_ih [N, 4H, I], weight_hh [N, 4H, H], biases [N, 4H]) the reference extracts at
    wide_lstm.py:184-199."""
    n, b, t, _ = x.shape
    h = weight_hh.shape[2]
    if hx is not None:
        h_t, c_t = hx
    else:
        h_t = x.new_zeros(n, b, h)
        c_t = x.new_zeros(n, b, h)
    gates_x = torch.einsum("nbti,ngi->nbtg", x, weight_ih)
    if bias_ih is not None:
        gates_x = gates_x + bias_ih.view(n, 4 * h).view(n, 1, 1, 4 * h)
    outs = []
    for step in range(t):
        gates_h = torch.einsum("nbh,ngh->nbg", h_t, weight_hh)
        if bias_hh is not None:
            gates_h = gates_h + bias_hh.view(n, 4 * h).view(n, 1, 4 * h)
        gates = gates_x[:, :, step, :] + gates_h
        i_g, f_g, g_g, o_g = gates.chunk(4, dim=-1)
        i_t = torch.sigmoid(i_g)
        f_t = torch.sigmoid(f_g)
        g_t = torch.tanh(g_g)
        o_t = torch.sigmoid(o_g)
        c_t = f_t * c_t + i_t * g_t
        h_t = o_t * torch.tanh(c_t)
        outs.append(h_t)
    return torch.stack(outs, dim=2), (h_t, c_t)


def attention(query: Tensor, key: Tensor, value: Tensor, q_weight: Tensor, kv_weight: Tensor,
              out_weight: Tensor, q_bias: Optional[Tensor], kv_bias: Optional[Tensor],
              out_bias: Optional[Tensor], n_heads: int, attn_mask: Optional[Tensor] = None,
              is_causal: bool = False) -> Tensor:
    """WideAttention._forward_fused, wide_attention.py:192-238 (eval: dropout 0)."""
    n, d = q_weight.shape[0], q_weight.shape[1]
    hh = n_heads
    dh = d // hh
    _, b, tq, _ = query.shape
    tkv = key.size(2)
    q = torch.einsum("nbtd,nod->nbto", query, q_weight)
    if q_bias is not None:
        q = q + q_bias.view(n, 1, 1, d)
    k = torch.einsum("nbtd,nod->nbto", key, kv_weight[:, :d, :])
    v = torch.einsum("nbtd,nod->nbto", value, kv_weight[:, d:, :])
    if kv_bias is not None:
        k = k + kv_bias[:, :d].view(n, 1, 1, d)
        v = v + kv_bias[:, d:].view(n, 1, 1, d)
    q = q.view(n, b, tq, hh, dh).permute(0, 1, 3, 2, 4).reshape(n * b, hh, tq, dh)
    k = k.view(n, b, tkv, hh, dh).permute(0, 1, 3, 2, 4).reshape(n * b, hh, tkv, dh)
    v = v.view(n, b, tkv, hh, dh).permute(0, 1, 3, 2, 4).reshape(n * b, hh, tkv, dh)
    o = F.scaled_dot_product_attention(q, k, v, attn_mask=attn_mask, dropout_p=0.0, is_causal=is_causal)
    o = o.view(n, b, hh, tq, dh).permute(0, 1, 3, 2, 4).reshape(n, b, tq, d)
    out = torch.einsum("nbtd,nod->nbto", o, out_weight)
    if out_bias is not None:
        out = out + out_bias.view(n, 1, 1, d)
    return out


# ---------------------------------------------------------------------------------------
# traced models of the benchmark configurations (cli.py:59-97) through the wide path
# ---------------------------------------------------------------------------------------

def mlp_wide(packed: Tensor, n: int, w1: Tensor, b1: Tensor, w2: Tensor, b2: Tensor) -> Tensor:
    """TracedWideModel over cli.py:59-67 (fc1 -> relu -> fc2), traced_wide.py:450-534."""
    x = to_nfirst(packed, n)
    h = F.relu(linear(x, w1, b1))
    return to_packed(linear(h, w2, b2))


def resblock_wide(packed: Tensor, n: int, p: dict) -> Tensor:
    """TracedWideModel over cli.py:84-97: relu(bn1(conv1 x)) -> bn2(conv2) -> + x -> relu."""
    x = to_nfirst(packed, n)
    out = conv2d(x, p["conv1.weight"], p["conv1.bias"], n, padding=(1, 1))
    out = batchnorm_eval(out, p["bn1.weight"], p["bn1.bias"], p["bn1.running_mean"], p["bn1.running_var"],
                         p["bn1.eps"], n)
    out = F.relu(out)
    out = conv2d(out, p["conv2.weight"], p["conv2.bias"], n, padding=(1, 1))
    out = batchnorm_eval(out, p["bn2.weight"], p["bn2.bias"], p["bn2.running_mean"], p["bn2.running_var"],
                         p["bn2.eps"], n)
    return to_packed(F.relu(out + x))


def seq_model(ids: Tensor, p: dict) -> Tensor:
    """Embedding -> LayerNorm -> LSTM -> Linear composed from the wide primitives, per-model ids
    [N, B, T]; returns logits [N, B, T, V]."""
    n = p["emb.weight"].shape[0]
    e = embedding_per_model(p["emb.weight"], ids)
    e = layernorm(e, p["ln.weight"], p["ln.bias"], n, p["ln.eps"])
    o, _ = lstm(e, p["lstm.weight_ih"], p["lstm.weight_hh"], p["lstm.bias_ih"], p["lstm.bias_hh"])
    return linear(o, p["fc.weight"], p["fc.bias"])
