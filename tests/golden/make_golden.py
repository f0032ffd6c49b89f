"""Write golden input/output vectors from the reference's own Python code.

Run once in the development container, where the read-only reference is
mounted (it never travels to the GPU machines):

    python tests/golden/make_golden.py /root/reference

Only numpy/torch modules of the reference are imported, each by file path:
  krunch_ac/cdf.py            probs_to_cdf             -> cdf_golden.npz
  krunch_ac/cpu_reference.py  encode / decode          -> rc_golden.npz
  krunch/batched_rwkv4.py     init_state_batched /
                              forward_batched          -> rwkv_golden.npz
The reference forward calls the third-party op `rwkv::wkv_forward`
(rwkv==0.8.26, not installed). It is registered here as a float64
implementation of the recurrence of krunch_ac/cuda/wkv_kernel.cu:52-73, so
the fixture pins the reference's layer code around the WKV; the WKV itself is
pinned separately by closed forms. Inputs are regenerated in the tests from
the seeds recorded here; large outputs are stored as SHA-256 digests.
"""
from __future__ import annotations

import hashlib
import importlib.util
import os
import sys
import types

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _load(ref_root, rel, name):
    spec = importlib.util.spec_from_file_location(name, os.path.join(ref_root, rel))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def rand_probs(N, V, seed):
    """Same construction as the reference tests (tests/test_ac_reference.py:14-18)."""
    rng = np.random.default_rng(seed)
    p = rng.random((N, V)).astype(np.float32)
    p /= p.sum(axis=1, keepdims=True)
    return p


def special_probs(kind, V):
    if kind == "peaky":
        p = np.full((1, V), 1e-9, dtype=np.float32)
        p[0, V // 2] = 1.0
    elif kind == "uniform":
        p = np.full((1, V), 1.0 / V, dtype=np.float32)
    elif kind == "ties":                      # two equal maxima: first index wins
        p = np.full((1, V), 1.0, dtype=np.float32)
        p[0, 3] = p[0, V - 2] = 50.0
    elif kind == "unnormalised":              # the spec renormalises
        p = np.arange(1, V + 1, dtype=np.float32).reshape(1, V)
    else:
        raise ValueError(kind)
    return p


CDF_CASES = [("rand", 1, 4, 10), ("rand", 16, 64, 11), ("rand", 8, 1000, 12),
             ("rand", 4, 8193, 13), ("rand", 2, 50277, 14), ("peaky", 1, 100, 0),
             ("uniform", 1, 50277, 0), ("ties", 1, 300, 0), ("unnormalised", 1, 777, 0)]


def case_probs(kind, N, V, seed):
    return rand_probs(N, V, seed) if kind == "rand" else special_probs(kind, V)


def sample_symbols(p, seed):
    rng = np.random.default_rng(seed + 100)
    cum = np.cumsum(p, axis=1)
    u = rng.random((p.shape[0], 1)).astype(np.float32)
    return np.minimum((u < cum).argmax(axis=1), p.shape[1] - 1).astype(np.int32)


RC_CASES = [(1, 4, 20), (8, 32, 21), (64, 256, 22), (300, 1000, 23), (40, 50277, 24)]

# tiny RWKV-4 for the forward fixture
TINY = dict(n_layer=2, C=32, F=128, V=67, B=2, T1=5, T2=3, seed=7)


def tiny_weights(n_layer, C, F, V, seed, **_):
    g = torch.Generator().manual_seed(seed)
    n = lambda *s: torch.randn(*s, generator=g) * 0.3
    u = lambda *s: torch.rand(*s, generator=g)
    w = {"emb.weight": n(V, C), "ln_out.weight": 1 + 0.2 * n(C), "ln_out.bias": 0.2 * n(C),
         "head.weight": n(C, V)}
    for i in range(n_layer):
        a, f, b = f"blocks.{i}.att.", f"blocks.{i}.ffn.", f"blocks.{i}."
        for k in ("key", "value", "receptance", "output"):
            w[a + k + ".weight"] = n(C, C)
        w[f + "key.weight"] = n(C, F)
        w[f + "receptance.weight"] = n(C, C)
        w[f + "value.weight"] = n(F, C)
        for k in ("time_mix_k", "time_mix_v", "time_mix_r"):
            w[a + k] = u(C)
        for k in ("time_mix_k", "time_mix_r"):
            w[f + k] = u(C)
        w[a + "time_decay"] = torch.linspace(-3.0, 1.0, C) + 0.1 * n(C)   # raw
        w[a + "time_first"] = 0.5 * n(C)
        for ln in ("ln1", "ln2"):
            w[b + ln + ".weight"] = 1 + 0.2 * n(C)
            w[b + ln + ".bias"] = 0.2 * n(C)
    return {k: v.float().contiguous() for k, v in w.items()}


def tiny_ids(V, B, T1, T2, seed, **_):
    rng = np.random.default_rng(seed)
    return rng.integers(0, V, size=(B, T1 + T2)).astype(np.int64)


def _register_wkv_op():
    def wkv(B, T, C, w, u, k, v, y, aa, bb, pp):
        w64, u64 = w.double(), u.double()
        a, b_, p = aa.double().view(B, C), bb.double().view(B, C), pp.double().view(B, C)
        k3, v3 = k.double().view(B, T, C), v.double().view(B, T, C)
        out = torch.empty(B, T, C, dtype=torch.float64)
        for t in range(T):
            kt, vt = k3[:, t], v3[:, t]
            ww = u64 + kt
            q = torch.maximum(p, ww)
            e1, e2 = torch.exp(p - q), torch.exp(ww - q)
            out[:, t] = (e1 * a + e2 * vt) / (e1 * b_ + e2)
            ww = w64 + p
            q = torch.maximum(ww, kt)
            e1, e2 = torch.exp(ww - q), torch.exp(kt - q)
            a, b_, p = e1 * a + e2 * vt, e1 * b_ + e2, q
        y.copy_(out.view_as(y).float())
        aa.copy_(a.view_as(aa).float())
        bb.copy_(b_.view_as(bb).float())
        pp.copy_(p.view_as(pp).float())

    lib = torch.library.Library("rwkv", "DEF")
    lib.define("wkv_forward(int B, int T, int C, Tensor w, Tensor u, Tensor k, Tensor v, "
               "Tensor(a!) y, Tensor(b!) aa, Tensor(c!) bb, Tensor(d!) pp) -> ()")
    lib.impl("wkv_forward", wkv, "CPU")
    return lib


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main(ref_root):
    cdf_mod = _load(ref_root, "krunch_ac/cdf.py", "ref_cdf")
    rc_mod = _load(ref_root, "krunch_ac/cpu_reference.py", "ref_cpu_reference")

    out = {}
    for idx, (kind, N, V, seed) in enumerate(CDF_CASES):
        cdf = cdf_mod.probs_to_cdf(case_probs(kind, N, V, seed))
        out[f"cdf{idx}_sha"] = np.array(digest(cdf.astype(np.uint32)))
        if cdf.size <= 20000:
            out[f"cdf{idx}"] = cdf.astype(np.uint32)
    out["cases"] = np.array([f"{k},{n},{v},{s}" for k, n, v, s in CDF_CASES])
    np.savez_compressed(os.path.join(HERE, "cdf_golden.npz"), **out)

    out = {}
    for idx, (N, V, seed) in enumerate(RC_CASES):
        p = rand_probs(N, V, seed)
        sym = sample_symbols(p, seed)
        cdf = cdf_mod.probs_to_cdf(p)
        bs = rc_mod.encode(cdf, sym)
        dec = rc_mod.decode(bs, cdf)
        assert (dec == sym).all()
        out[f"bits{idx}"] = np.frombuffer(bs, dtype=np.uint8)
        out[f"sym{idx}"] = sym
        out[f"cdf{idx}_sha"] = np.array(digest(cdf.astype(np.uint32)))
    out["cases"] = np.array(RC_CASES)
    np.savez_compressed(os.path.join(HERE, "rc_golden.npz"), **out)

    lib = _register_wkv_op()  # noqa: F841  (keeps the op registered)
    br = _load(ref_root, "krunch/batched_rwkv4.py", "ref_batched_rwkv4")
    os.environ.pop("KRUNCH_PURE_WKV", None)
    os.environ.pop("KRUNCH_PLAIN_MATMUL", None)
    w_raw = tiny_weights(**TINY)
    w_model = dict(w_raw)
    for i in range(TINY["n_layer"]):
        key = f"blocks.{i}.att.time_decay"
        w_model[key] = -torch.exp(w_raw[key])      # the rwkv loader's conversion
    m = types.SimpleNamespace(
        version=4, w=w_model,
        args=types.SimpleNamespace(n_layer=TINY["n_layer"], n_embd=TINY["C"], n_att=TINY["C"]),
        strategy=[types.SimpleNamespace(atype=torch.float32, device=torch.device("cpu"))
                  for _ in range(TINY["n_layer"])])
    ids = tiny_ids(**TINY)
    state = br.init_state_batched(m, TINY["B"], device="cpu")
    with torch.no_grad():
        l1, state = br.forward_batched(m, torch.as_tensor(ids[:, :TINY["T1"]]), state)
        l2, state = br.forward_batched(m, torch.as_tensor(ids[:, TINY["T1"]:]), state)
    out = {"logits_w1": l1.numpy(), "logits_w2": l2.numpy(), "ids": ids,
           "state": torch.stack([s.float() for s in state]).numpy()}
    np.savez_compressed(os.path.join(HERE, "rwkv_golden.npz"), **out)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
