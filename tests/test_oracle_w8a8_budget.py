"""Where the w8a8 codec's distance from the fp32 logits comes from, on the
BASELINE weights (random init, N(0, 0.02) matrices), in the oracle's exact
arithmetic (no fp16 rounding).

north_star asks int8 logits within 5e-2 max-abs of fp32; the scheme that
BASELINE config 4 prescribes (symmetric per-output-channel int8 weights,
per-token dynamic int8 activations) lands at ~0.13. These tests pin the
budget behind that figure: quantising the weights alone, with every
activation exact, already moves the logits by more than 5e-2, and so does
quantising the activations alone. So no activation-side change (smoothing,
rotation, clipping of activations) can meet 5e-2 while the weights are
per-channel int8 rounded to nearest. Nothing here touches the GPU.
"""
import numpy as np
import pytest
import torch

from krunch_amd import synthetic
from oracle import quant, rwkv4

B, T = 1, 16
PRODUCTS = {"att.key": "K", "att.value": "V", "att.receptance": "R", "att.output": "O",
            "ffn.key": "fK", "ffn.receptance": "fR", "ffn.value": "fV"}


def _qdq(x: np.ndarray) -> np.ndarray:
    """x rounded to the int8 grid of its rows (oracle.quant's rule), as float64."""
    q, s = quant.quantize_rows(x.astype(np.float32))
    return q.astype(np.float64) * s.astype(np.float64)[:, None]


@pytest.fixture(scope="module")
def setup():
    torch.set_num_threads(min(8, torch.get_num_threads()))
    w = {k: v.float() for k, v in synthetic.make_weights().items()}
    tag = {id(v): p for k, v in w.items() for n, p in PRODUCTS.items() if k.endswith(n + ".weight")}
    ids = torch.as_tensor(synthetic.model_inputs(synthetic.zipf_tokens(B, T)))
    return w, tag, ids


def _logits(setup, monkeypatch, mode: str, only=None) -> np.ndarray:
    """mode: "" fp32, "w" weights int8, "a" activations int8, "wa" both;
    only: restrict the quantisation to one product tag."""
    w, tag, ids = setup

    def mm(x, W, rowwise, q8=False):
        p = tag.get(id(W))
        X = x.reshape(-1, x.shape[-1]).numpy().astype(np.float64)
        Wn = W.numpy().astype(np.float64)
        if p is not None and (only is None or p == only):
            if "a" in mode:
                X = _qdq(X)
            if "w" in mode:
                Wn = _qdq(Wn.T).T
        y = torch.from_numpy(X @ Wn).float()
        return y.reshape(*x.shape[:-1], W.shape[-1])

    monkeypatch.setattr(rwkv4, "_mm", mm)
    return rwkv4.forward(w, ids, rwkv4.new_state(12, B, 768)).numpy()


def test_weight_and_activation_shares_each_exceed_the_tolerance(setup, monkeypatch):
    """The int8 oracle (integer products, float32 scales) and the scheme's
    products in float64 (operands rounded to the int8 grid) both land
    between 5e-2 and 0.2. They are not equal bit for bit: a last-place
    difference upstream can move an activation across an int8 rounding
    boundary, which then shifts later logits by a few 1e-2."""
    w, _, ids = setup
    f32 = _logits(setup, monkeypatch, "")
    err = {m: np.abs(_logits(setup, monkeypatch, m) - f32).max() for m in ("wa", "w", "a")}
    monkeypatch.undo()
    q8 = rwkv4.forward(w, ids, rwkv4.new_state(12, B, 768), w8a8=True).numpy()
    err["int8 oracle"] = np.abs(q8 - f32).max()
    # the whole scheme, its weights alone and its activations alone
    assert 5e-2 < err["int8 oracle"] < 0.2, err
    assert 5e-2 < err["wa"] < 0.2, err
    assert err["w"] > 5e-2, err
    assert err["a"] > 5e-2, err


def test_value_product_activation_is_the_largest_single_share(setup, monkeypatch):
    """The ReLU^2 operand of the channel-mix value product is heavy-tailed
    (row max ~10x its rms), so its per-token int8 grid is the coarsest; the
    K, R and channel-mix R products contribute least."""
    f32 = _logits(setup, monkeypatch, "")
    share = {p: np.abs(_logits(setup, monkeypatch, "a", p) - f32).max()
             for p in ("K", "R", "fR", "fV")}
    assert share["fV"] == max(share.values()), share
    assert max(share["K"], share["R"], share["fR"]) < share["fV"] / 2, share
