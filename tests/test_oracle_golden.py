"""Pin the oracle against vectors written by the reference's own code
(tests/golden/make_golden.py): krunch_ac/cdf.py, krunch_ac/cpu_reference.py,
krunch/batched_rwkv4.py."""
import hashlib
import os

import numpy as np
import torch

from oracle import cdf as ocdf
from oracle import range_coder as orc
from oracle import rwkv4
from tests.golden import make_golden as mg


def _load(golden_dir, name):
    return np.load(os.path.join(golden_dir, name), allow_pickle=False)


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a.astype(np.uint32)).tobytes()).hexdigest()


def test_probs_to_cdf_matches_reference(golden_dir):
    g = _load(golden_dir, "cdf_golden.npz")
    for idx, (kind, N, V, seed) in enumerate(mg.CDF_CASES):
        cdf = ocdf.probs_to_cdf(mg.case_probs(kind, N, V, seed))
        assert _sha(cdf) == str(g[f"cdf{idx}_sha"]), (kind, N, V)
        if f"cdf{idx}" in g:
            np.testing.assert_array_equal(cdf, g[f"cdf{idx}"])


def test_encode_matches_reference_bitstreams(golden_dir):
    g = _load(golden_dir, "rc_golden.npz")
    for idx, (N, V, seed) in enumerate(mg.RC_CASES):
        p = mg.rand_probs(N, V, seed)
        sym = mg.sample_symbols(p, seed)
        np.testing.assert_array_equal(sym, g[f"sym{idx}"])
        cdf = ocdf.probs_to_cdf(p)
        assert _sha(cdf) == str(g[f"cdf{idx}_sha"])
        bits = orc.encode(cdf, sym)
        assert bits == g[f"bits{idx}"].tobytes(), (N, V)
        np.testing.assert_array_equal(orc.decode(bits, cdf), sym)


def test_forward_matches_reference_layer_code(golden_dir):
    g = _load(golden_dir, "rwkv_golden.npz")
    t = mg.TINY
    w = mg.tiny_weights(**t)
    ids = mg.tiny_ids(**t)
    np.testing.assert_array_equal(ids, g["ids"])
    st = rwkv4.new_state(t["n_layer"], t["B"], t["C"])
    l1 = rwkv4.forward(w, torch.as_tensor(ids[:, :t["T1"]]), st)
    l2 = rwkv4.forward(w, torch.as_tensor(ids[:, t["T1"]:]), st)
    np.testing.assert_allclose(l1.numpy(), g["logits_w1"], atol=2e-4, rtol=1e-4)
    np.testing.assert_allclose(l2.numpy(), g["logits_w2"], atol=2e-4, rtol=1e-4)
    ref_state = g["state"]
    for i, s in enumerate(st):
        for j, key in enumerate(("att_xx", "aa", "bb", "pp", "ffn_xx")):
            np.testing.assert_allclose(s[key].numpy(), ref_state[5 * i + j],
                                       atol=2e-4, rtol=1e-4, err_msg=f"layer {i} {key}")
