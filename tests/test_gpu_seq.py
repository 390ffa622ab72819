"""GPU parity of the composed sequence model (per-model Embedding -> LayerNorm -> LSTM -> Linear)
and of the streamed large-hidden LSTM recurrence against the oracle."""

import pytest
import torch

from oracle import wide_ref
from tests._util import TOL_BF16, gen, rel_err, tol

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _models(n, v, d, h, dtype, seed=500):
    from wide_compiler.workloads import SeqModel
    mods = []
    for i in range(n):
        torch.manual_seed(seed + i)
        m = SeqModel(v, d, h)
        with torch.no_grad():
            m.ln.weight.normal_(1.0, 0.2)
            m.ln.bias.normal_(0.0, 0.2)
        mods.append(m.to(dtype).eval())
    return mods


def _exact(mods, ids):
    from wide_compiler.workloads import seq_params
    p = {k: (v.double() if torch.is_tensor(v) else v) for k, v in seq_params(mods).items()}
    return wide_ref.seq_model(ids, p)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,b,t,v,d,h", [(3, 2, 5, 64, 32, 64),      # register-resident recurrence
                                         (2, 3, 4, 96, 64, 512)])    # streamed recurrence
def test_seq_model(hip, dtype, n, b, t, v, d, h):
    from wide_compiler.workloads import WideSeqModel
    mods = _models(n, v, d, h, dtype)
    ids = torch.randint(0, v, (n, b, t), generator=gen(501))
    wide = WideSeqModel([m.to(DEV) for m in mods])
    with torch.no_grad():
        y = wide(ids.to(DEV)).cpu()
    wide.emb.index_error()
    exact = _exact([m.cpu() for m in mods], ids)
    assert y.shape == exact.shape
    assert rel_err(y, exact) <= tol(dtype)


def test_embedding_strict_ids_raise_at_the_call(hip):
    """strict_ids = True: an out-of-range id raises IndexError from the forward itself, as the
    reference's weight[:, ids] does; in-range ids pass and the flag starts clear."""
    import wide_compiler as wc
    emb = wc.WideEmbedding.from_modules([torch.nn.Embedding(10, 8) for _ in range(3)]).to(DEV)
    emb.strict_ids = True
    with torch.no_grad():
        emb(torch.tensor([[1, 9], [0, 3]], device=DEV))
        with pytest.raises(IndexError):
            emb(torch.tensor([[1, 10], [0, 3]], device=DEV))
        with pytest.raises(IndexError):
            emb(torch.tensor([[-1, 2], [0, 3], [4, 5]], device=DEV), per_model=True)
        y = emb(torch.tensor([[2, 3]], device=DEV))      # the flag was cleared by the raise
    assert y.shape == (3, 1, 2, 8)


def test_seq_model_out_of_range_id_raises(hip):
    from wide_compiler.workloads import WideSeqModel
    mods = _models(2, 16, 8, 32, torch.float32)
    ids = torch.randint(0, 16, (2, 2, 3), generator=gen(502))
    ids[1, 0, 2] = 16
    wide = WideSeqModel([m.to(DEV) for m in mods])
    with torch.no_grad():
        wide(ids.to(DEV))
    with pytest.raises(IndexError):
        wide.emb.index_error()


# Per-timestep bar of the recurrent outputs (LSTM output at every t, final cell state)
# against the reference's own bf16 path: that path keeps its cell state and gates in bf16
# and drifts up to ~0.02 from fp64 itself (measured ~0.016-0.02 per timestep on this
# configuration), while this build stays within ~0.006 of fp64; two approximations on
# either side of the exact answer can differ by the sum, so the bar is 3e-2 per timestep.
# The logits are not a recurrent output: they are held to the bf16 bar (2e-2) against
# fp64, against the reference's bf16 path end to end, and against the reference's bf16
# Linear applied to this build's own LSTM output.
TOL_BF16_PATH = 3e-2


def test_seq_config_n64(hip):
    """The sequence configuration at full size: N=64, B=16, T=128, vocab 8192, 256 -> 512, bf16,
    through WideSeqModel.forward (the launches the benchmark times: gather with the LayerNorm
    applied as rows are gathered, partitioned LSTM, vocabulary GEMM), which also returns the
    LSTM output and state.  Every model (the wide path has no cross-model terms) against the
    fp64 oracle (2e-2 at every timestep of the LSTM output, the final cell state and the
    logits) and against the reference's own bf16 path (bf16 gates and bf16 cell state,
    wide_lstm.py:205-229; recurrent outputs 3e-2 per timestep, TOL_BF16_PATH; logits 2e-2);
    the bf16 path's own distance from fp64 is checked too."""
    from wide_compiler.workloads import WideSeqModel, seq_n64, seq_params
    wl = seq_n64()
    ids = wl.inputs["ids"]
    wide = WideSeqModel([m.to(DEV) for m in wl.models])
    with torch.no_grad():
        y, hs, (hn, cn) = wide(ids.to(DEV), return_state=True)
    hip.rnn_sync_check(block=True)
    wide.emb.index_error()
    assert y.shape == (64, 16, 128, 8192) and hs.shape == (64, 16, 128, 512)
    worst = {"h fp64": 0.0, "h bf16 path": 0.0, "h bf16 path vs fp64": 0.0,
             "logits fp64": 0.0, "logits bf16 path": 0.0, "logits bf16 linear of own h": 0.0}
    for k in range(64):
        pb = seq_params([wl.models[k].cpu()])
        pd = {kk: (vv.double() if torch.is_tensor(vv) else vv) for kk, vv in pb.items()}
        got_h, got_c, got_y = hs[k:k + 1].cpu(), cn[k:k + 1].cpu(), y[k:k + 1].cpu()
        ref = {}
        for name, p in (("fp64", pd), ("bf16 path", pb)):
            e = wide_ref.layernorm(wide_ref.embedding_per_model(p["emb.weight"], ids[k:k + 1]), p["ln.weight"],
                                   p["ln.bias"], 1, p["ln.eps"])
            eo, (eh, ec) = wide_ref.lstm(e, p["lstm.weight_ih"], p["lstm.weight_hh"], p["lstm.bias_ih"],
                                         p["lstm.bias_hh"])
            ref[name] = eo
            bar = TOL_BF16 if name == "fp64" else TOL_BF16_PATH
            step_err = max(rel_err(got_h[:, :, s], eo[:, :, s]) for s in range(128))
            worst["h " + name] = max(worst["h " + name], step_err)
            assert step_err <= bar, (k, name, step_err)
            assert rel_err(got_c, ec) <= bar, (k, name)
            y_err = rel_err(got_y, wide_ref.linear(eo, p["fc.weight"], p["fc.bias"]))
            worst["logits " + name] = max(worst["logits " + name], y_err)
            assert y_err <= TOL_BF16, (k, name, y_err)
        own = rel_err(got_y, wide_ref.linear(got_h, pb["fc.weight"], pb["fc.bias"]))
        worst["logits bf16 linear of own h"] = max(worst["logits bf16 linear of own h"], own)
        assert own <= TOL_BF16, (k, own)
        drift = max(rel_err(ref["bf16 path"][:, :, s], ref["fp64"][:, :, s]) for s in range(128))
        worst["h bf16 path vs fp64"] = max(worst["h bf16 path vs fp64"], drift)
    print("worst errors over the 64 models", worst)
