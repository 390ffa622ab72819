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


def test_seq_config_n64(hip):
    """The sequence configuration at full size: N=64, B=16, T=128, vocab 8192, 256 -> 512, bf16.
    Checked model-by-model on three models (the wide path has no cross-model terms), with the
    LSTM output compared per timestep."""
    from wide_compiler.workloads import WideSeqModel, seq_n64
    wl = seq_n64()
    ids = wl.inputs["ids"]
    wide = WideSeqModel([m.to(DEV) for m in wl.models])
    with torch.no_grad():
        x = wide.ln(wide.emb(ids.to(DEV), per_model=True))
        hs, (hn, cn) = wide.lstm(x)
        y = wide.fc(hs)
    wide.emb.index_error()
    assert y.shape == (64, 16, 128, 8192)
    for k in (0, 37, 63):
        m = wl.models[k].cpu()
        exact = _exact([m], ids[k:k + 1])
        assert rel_err(y[k:k + 1].cpu(), exact) <= TOL_BF16
        from wide_compiler.workloads import seq_params
        p = {kk: (vv.double() if torch.is_tensor(vv) else vv) for kk, vv in seq_params([m]).items()}
        e = wide_ref.layernorm(wide_ref.embedding_per_model(p["emb.weight"], ids[k:k + 1]), p["ln.weight"],
                               p["ln.bias"], 1, p["ln.eps"])
        eo, (eh, ec) = wide_ref.lstm(e, p["lstm.weight_ih"], p["lstm.weight_hh"], p["lstm.bias_ih"],
                                     p["lstm.bias_hh"])
        got = hs[k:k + 1].cpu()
        errs = [rel_err(got[:, :, s], eo[:, :, s]) for s in range(128)]
        assert max(errs) <= TOL_BF16, max(errs)
        assert rel_err(cn[k:k + 1].cpu(), ec) <= TOL_BF16
