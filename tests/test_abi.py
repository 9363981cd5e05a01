"""The C-ABI library loads and exports every entry point declared in include/*.h (no GPU
calls here), and the Python binding covers the same set."""

import ctypes
import re
from pathlib import Path

REPO = Path(__file__).resolve().parents[1]


def _declared():
    names = set()
    for h in (REPO / "include").glob("*.h"):
        txt = h.read_text()
        txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
        names |= set(re.findall(r"\b(dsk_[a-z0-9_]+)\s*\(", txt))
    return names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(REPO / "mlx-dspark_amd" / "mlx_dspark" / "libdspark_hip.so"))
    declared = _declared()
    assert declared, "no declarations found"
    missing = [n for n in sorted(declared) if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_matches_header():
    from mlx_dspark import _hip
    assert set(_hip.SIGNATURES) == _declared()
    assert _hip.lib.dsk_abi_version() == 1


def test_size_queries_without_gpu():
    from mlx_dspark import _hip
    assert _hip.lib.dsk_act_pack_bytes(16, 4096) == 16 * 4096 * 2
    assert _hip.lib.dsk_act_pack_bytes(17, 4096) == 32 * 4096 * 2
    assert _hip.lib.dsk_act_pack_bytes(0, 64) == 0 and _hip.lib.dsk_act_pack_bytes(4, 96) == 0
    assert 1 <= _hip.lib.dsk_w8_gemm_splits(16, 4096, 4096) <= 16
    assert _hip.lib.dsk_w8_gemm_splits(16, 4096, 4000) == 0
    assert 1 <= _hip.lib.dsk_w4_gemm_splits(16, 4096, 4096) <= 16
    assert _hip.lib.dsk_w4_gemm_splits(65, 4096, 4096) == 0
    assert _hip.lib.dsk_argmax_ws_bytes(15) >= 4096 + 2 * 15 * 16 * 4
    assert _hip.lib.dsk_argmax_ws_bytes(0) == 0 and _hip.lib.dsk_argmax_ws_bytes(1025) == 0
    # sampled acceptance: one candidate key per vocabulary entry for each of the B * (2L + 1) rows
    assert _hip.lib.dsk_accept_ws_bytes(4, 17, 151936) >= 4 * 33 * 151936 * 4
    assert _hip.lib.dsk_sample_ws_bytes(15, 151936) >= 15 * 151936 * 4
    assert _hip.lib.dsk_sample_ws_bytes(0, 151936) == 0


def test_error_path_reports_message():
    from mlx_dspark import _hip
    rc = _hip.lib.dsk_w8_quantize(None, 0, 16, 64, None, None, None, None)
    assert rc == -1
    assert b"null pointer" in _hip.lib.dsk_last_error()


def test_gemm_plan_query_names_the_traced_kernels():
    # the verify step's GEMMs at 16 rows, named as the kernel trace of the Qwen3-8B verify forward
    # names them (w8_gemm_kernel<row tiles, slab tiles, batch groups, waves, epilogue, pipelined, bits>)
    from mlx_dspark import ops
    P, R, SW, ST = ops.DSK_EPI_PARTIAL, ops.DSK_EPI_RESIDUAL, ops.DSK_EPI_SWIGLU, ops.DSK_EPI_STORE
    want = {(6144, 4096, P, False): "w8_gemm_kernel<1, 3, 2, 16, 2, false, 8>",
            (4096, 4096, R, False): "w8_gemm_kernel<1, 1, 2, 16, 3, true, 8>",
            (24576, 4096, SW, True): "w8_gemm_kernel<1, 2, 2, 8, 5, false, 8>",
            (4096, 12288, R, False): "w8_gemm_kernel<1, 1, 2, 8, 3, false, 8>",
            (151936, 4096, ST, True): "w8_gemm_kernel<1, 4, 2, 8, 4, false, 8>"}
    for (N, K, epi, rs), name in want.items():
        assert ops.gemm_kernel_name(16, N, K, epi, rs) == name
    assert ops.gemm_plan(16, 4096, 4096, R)[3] == 1            # the residual epilogue never splits K
    import pytest
    with pytest.raises(RuntimeError):
        ops.gemm_plan(16, 4096, 4000, R)
