"""Drop-in for the reference's `krunch.batched_rwkv4` entry points
(`init_state_batched`, `forward_batched`; `krunch/batched_rwkv4.py:60-262`),
running every layer through the HIP library.

`m` is duck-typed as in the reference: `m.w` (rwkv-package keys, [in,out]
matrices, raw time_decay), `m.args.n_layer/n_embd/n_att`, `m.version == 4`.
State is the reference's flat list: per layer [att_xx fp16, aa, bb, pp fp32,
ffn_xx fp16], each [B, C]. Logits are fp16 (the reference's fp16 strategy).
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import torch

from krunch_amd import _lib, cpp_path


class _StateList(list):
    """The flat state list; keeps the owning device buffer alive."""
    owner = None


def init_state_batched(m, B: int, device="cuda") -> List[torch.Tensor]:
    weights = cpp_path.init_weights(m, device)
    st = cpp_path.fresh_state_batched(weights, B)
    out = _StateList(st.flat())
    out.owner = st
    return out


def forward_batched(m, tokens_batches, state: Optional[List[torch.Tensor]] = None,
                    full_output: bool = True) -> Tuple[torch.Tensor, List[torch.Tensor]]:
    assert getattr(m, "version", 4) == 4, "batched forward implemented for v4 only"
    weights = cpp_path.init_weights(m, "cuda")
    P = weights["prepared"]
    if isinstance(tokens_batches, torch.Tensor):
        idx = tokens_batches.to(device=P.device, dtype=torch.int32)
        if idx.dim() == 1:
            idx = idx.unsqueeze(1)
    else:
        T0 = len(tokens_batches[0])
        assert all(len(b) == T0 for b in tokens_batches), "streams must share T (caller pads)"
        idx = torch.as_tensor(tokens_batches, dtype=torch.int32, device=P.device)
    idx = idx.contiguous()
    B, T = idx.shape
    cpp_path._check_ids(idx, P.V)
    if state is None:
        state = init_state_batched(m, B)
    assert len(state) == 5 * P.n_layer
    M = B * T
    s = _lib.stream_ptr()
    x = torch.empty((M, P.C), dtype=torch.float16, device=P.device)
    _lib.call("kr_embed", P.ptr, idx.data_ptr(), M, x.data_ptr(), s)
    ws, nbytes = cpp_path.workspace(weights, M)
    for i in range(P.n_layer):
        att_xx, aa, bb, pp, ffn_xx = state[5 * i:5 * i + 5]
        for t, dt in ((att_xx, torch.float16), (aa, torch.float32), (bb, torch.float32),
                      (pp, torch.float32), (ffn_xx, torch.float16)):
            assert t.dtype == dt and t.is_contiguous() and t.shape == (B, P.C), "bad state tensor"
        _lib.call("kr_layer_step", P.layer_ptr(i), P.C, P.F, x.data_ptr(), B, T,
                  att_xx.data_ptr(), aa.data_ptr(), bb.data_ptr(), pp.data_ptr(),
                  ffn_xx.data_ptr(), ws.data_ptr(), nbytes, s)
    if not full_output:
        x = x.view(B, T, P.C)[:, -1, :].contiguous()
        M = B
    xn = torch.empty_like(x)
    logits = torch.empty((M, P.V), dtype=torch.float16, device=P.device)
    _lib.call("kr_head_logits", P.ptr, x.data_ptr(), M, xn.data_ptr(), logits.data_ptr(), P.V, s)
    logits = logits.view(B, T, P.V) if full_output else logits.view(B, P.V)
    return logits, state
