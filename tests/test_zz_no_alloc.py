"""kr_layer_step_noalloc, the allocation-free layer step (its workspace is a
static device array), against kr_layer_step with a caller workspace: same
x and state bits on two calls in a row, the second with a smaller input,
state carried between them; sizes past the static scratch are refused."""
import ctypes

import pytest
import torch

from krunch_amd import _lib, cpp_path, synthetic

pytestmark = pytest.mark.gpu


def _layer_call(P, layer, x, B, T, st, noalloc, ws=None, nbytes=0):
    att_xx, aa, bb, pp, ffn_xx = st._layer(layer)
    args = [P.layer_ptr(layer), P.C, P.F, x.data_ptr(), B, T, att_xx.data_ptr(), aa.data_ptr(),
            bb.data_ptr(), pp.data_ptr(), ffn_xx.data_ptr()]
    if noalloc:
        return _lib.lib().kr_layer_step_noalloc(*args, _lib.stream_ptr())
    return _lib.lib().kr_layer_step(*args, ws.data_ptr(), nbytes, _lib.stream_ptr())


def test_noalloc_layer_step_matches_workspace_entry_point():
    W = cpp_path.init_weights(synthetic.make_weights(), "cuda")
    P = W["prepared"]
    B, layer = 8, 4
    st_ws = cpp_path.fresh_state_batched(W, B)
    st_na = cpp_path.fresh_state_batched(W, B)
    g = torch.Generator().manual_seed(7)
    # 1024 rows (the static scratch's limit at this shape, the large-M path),
    # then one token per stream (8 rows, the fused stepped path)
    for T in (128, 1):
        x = (torch.randn(B * T, P.C, generator=g) * 0.5).half().cuda()
        xa, xb = x.clone(), x.clone()
        nbytes = _lib.lib().kr_forward_workspace_bytes(B * T, P.C, P.F)
        assert nbytes <= _lib.NOALLOC_SCRATCH_BYTES
        ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        assert _layer_call(P, layer, xa, B, T, st_ws, False, ws, nbytes) == 0
        rc = _layer_call(P, layer, xb, B, T, st_na, True)
        assert rc == 0, _lib.lib().kr_last_error()
        torch.cuda.synchronize()
        assert torch.equal(xa, xb), f"T={T}: x differs"
        assert torch.equal(st_ws.buf, st_na.buf), f"T={T}: state differs"
        del ws


def test_noalloc_refuses_more_than_the_static_scratch():
    W = cpp_path.init_weights(synthetic.make_weights(), "cuda")
    P = W["prepared"]
    B, T = 1025, 1
    st = cpp_path.fresh_state_batched(W, B)
    x = torch.zeros(B * T, P.C, dtype=torch.float16, device="cuda")
    before = st.buf.clone()
    rc = _layer_call(P, 0, x, B, T, st, True)
    assert rc != 0
    assert b"static scratch" in _lib.lib().kr_last_error()
    torch.cuda.synchronize()
    assert torch.equal(st.buf, before) and not x.any()
