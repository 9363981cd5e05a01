"""GPU: the no-allocation greedy acceptance (dsk_accept_greedy_static, slice partials in a
file-scope device array) gives exactly what dsk_accept_greedy gives with a caller workspace,
called through the C ABI twice in a row (the second call smaller, so it runs over the first
call's leftovers in the shared array), plus the documented range
error (a host-side check, run without a GPU)."""

import ctypes as C

import numpy as np
import pytest
import torch


def _case(rng, B, W, V, dtype, dev):
    logits = rng.integers(-3, 4, size=(B, W, V)).astype(np.float32)   # plenty of exact ties
    tt = logits.argmax(axis=2)
    draft = tt[:, : W - 1].copy().astype(np.int32)
    for b in range(B):
        k = int(rng.integers(0, W))
        if k < W - 1:
            draft[b, k] = (draft[b, k] + 1) % V
    lt = torch.from_numpy(logits).to(dev)
    if dtype == "bf16":
        lt = lt.to(torch.bfloat16)
    sl = torch.from_numpy(rng.integers(0, 1000, size=B).astype(np.int32)).to(dev)
    return lt, torch.from_numpy(draft).to(dev), sl


def _static(lt, draft, sl):
    from mlx_dspark import _hip
    B, W, V = lt.shape
    dev = lt.device
    tt = torch.full((B, W), -7, dtype=torch.int32, device=dev)
    n = torch.full((B,), -7, dtype=torch.int32, device=dev)
    tok = torch.full((B,), -7, dtype=torch.int32, device=dev)
    dt = _hip.DSK_BF16 if lt.dtype == torch.bfloat16 else _hip.DSK_F32
    rc = _hip.lib.dsk_accept_greedy_static(_hip.ptr(lt), dt, V, B, W, V, _hip.ptr(draft), _hip.ptr(tt),
                                           _hip.ptr(n), _hip.ptr(tok), _hip.ptr(sl), _hip.stream_ptr())
    _hip.check(rc, "dsk_accept_greedy_static")
    return tt, n, tok


@pytest.mark.gpu
def test_static_greedy_matches_workspace_entry(dev):
    from mlx_dspark.ops import accept_greedy
    rng = np.random.default_rng(11)
    for B, W, V, dtype in [(8, 16, 151936, "f32"), (3, 5, 4099, "bf16")]:   # second call smaller
        print(f"static greedy B={B} W={W} V={V} {dtype}", flush=True)
        lt, draft, sl = _case(rng, B, W, V, dtype, dev)
        sl_ws, sl_st = sl.clone(), sl.clone()
        tt_w, n_w, tok_w = accept_greedy(lt, draft, seq_lens=sl_ws)
        tt_s, n_s, tok_s = _static(lt, draft, sl_st)
        torch.cuda.synchronize()
        assert torch.equal(tt_s, tt_w)
        assert torch.equal(n_s, n_w)
        assert torch.equal(tok_s, tok_w)
        assert torch.equal(sl_st, sl_ws)
        assert torch.equal(sl_st, sl + n_w + 1)


def test_static_greedy_rejects_rows_beyond_maximum():
    from mlx_dspark import _hip
    # host-side check: nothing is launched (null tensors would fault a kernel, so none runs)
    rc = _hip.lib.dsk_accept_greedy_static(C.c_void_p(16), _hip.DSK_F32, 1000, 65, 16, 1000, C.c_void_p(16),
                                           None, C.c_void_p(16), C.c_void_p(16), None, None)
    assert rc == -3
    assert b"beyond the static scratch maximum" in _hip.lib.dsk_last_error()
