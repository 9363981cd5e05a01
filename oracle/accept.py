"""Acceptance / sampling oracle: ctypes wrapper over accept_oracle.c plus a float64
restatement of the reference's sort-and-cumsum truncation used to pin the C version.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Reference functions restated: truncate_probs / sample_probs (src/mlx_dspark/sampling.py:18-49),
_spec_sample_accept (src/mlx_dspark/generate.py:659-688), fused greedy accept
(src/mlx_dspark/generate.py:910-921, :557-568; src/mlx_dspark/batch_engine.py:573-579).

Pinning:
  - Philox4x32-10 against the Random123 known-answer vectors;
  - oracle_expf against libm exp (ulp bound) over the softmax input range;
  - probs() against truncate_probs_ref() (float64 sort + cumsum, the reference's algorithm)
    on rows without near-ties at the nucleus boundary;
  - the top-p target ceil(top_p * Z) against exact rational arithmetic, and the order-free
    threshold rule the GPU uses (keep e >= max(k-th largest, nucleus cutoff of the untruncated
    row)) against the sequential top-k-then-top-p of probs() on tie-heavy rows;
  - losslessness: the exact output distribution of one accept step (computed from the
    oracle's p and q) equals truncate(softmax(target / T)), and the statistical KAT of
    tests/test_generate_helpers.py:145-170 in the reference replays within 0.02;
  - greedy accept against brute force over all draft/target patterns at tiny V.
"""

from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

_LIB = Path(__file__).with_name("liboracle.so")
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not _LIB.exists():
            raise ImportError(f"{_LIB} missing: run `python mlx-dspark_amd/build.py --oracle`")
        L = C.CDLL(str(_LIB))
        vp, i32, i64, f32, u64, u32 = C.c_void_p, C.c_int, C.c_int64, C.c_float, C.c_uint64, C.c_uint32
        L.oracle_philox.argtypes = [vp, u32, u32, vp]
        L.oracle_expf.argtypes = [f32]
        L.oracle_expf.restype = f32
        L.oracle_probs.argtypes = [vp, i64, f32, i32, f32, i32, vp]
        L.oracle_top_p_target.argtypes = [f32, u64]
        L.oracle_top_p_target.restype = u64
        L.oracle_categorical.argtypes = [vp, i64, u32]
        L.oracle_categorical.restype = i64
        L.oracle_accept_sample.argtypes = [vp, vp, i64, i32, i32, vp, f32, f32, i32, i32, u64, u32,
                                           vp, vp, vp, vp, vp]
        L.oracle_accept_greedy.argtypes = [vp, i32, i64, i32, i32, i64, vp, vp, vp, vp, vp]
        L.oracle_sample_rows.argtypes = [vp, i64, i32, f32, f32, i32, i32, u64, u32, i32, vp, vp]
        L.oracle_threads.restype = i32
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def threads() -> int:
    """Threads the sampled acceptance spreads its (row, position) items over (OpenMP)."""
    return int(lib().oracle_threads())


def philox(ctr, key):
    c = np.asarray(ctr, dtype=np.uint32)
    out = np.zeros(4, dtype=np.uint32)
    lib().oracle_philox(_p(c), int(key[0]), int(key[1]), _p(out))
    return out


def expf(x: float) -> float:
    return lib().oracle_expf(float(x))


def probs(logits: np.ndarray, T: float, top_p: float = 1.0, top_k: int = 0, mul_inv: bool = False):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    out = np.empty_like(logits)
    lib().oracle_probs(_p(logits), logits.size, T, int(mul_inv), top_p, int(top_k), _p(out))
    return out


def top_p_target(top_p: float, Z: int) -> int:
    return int(lib().oracle_top_p_target(float(top_p), int(Z)))


def categorical(w: np.ndarray, word: int) -> int:
    w = np.ascontiguousarray(w, dtype=np.float32)
    return int(lib().oracle_categorical(_p(w), w.size, int(word) & 0xFFFFFFFF))


def accept_sample(p_logits, q_logits, draft, T, top_p=1.0, top_k=0, q_mul_inv_t=False, seed=0,
                  offset=0, seq_lens=None):
    p_logits = np.ascontiguousarray(p_logits, dtype=np.float32)
    B, R, V = p_logits.shape
    L = R - 1
    ql = None if q_logits is None else np.ascontiguousarray(q_logits, dtype=np.float32)
    draft = np.ascontiguousarray(draft, dtype=np.int32).reshape(B, L)
    n = np.zeros(B, np.int32)
    tok = np.zeros(B, np.int32)
    acc = np.zeros((B, max(L, 1)), np.uint8)
    samp = np.zeros((B, R), np.int32)
    sl = None if seq_lens is None else np.ascontiguousarray(seq_lens, dtype=np.int32).copy()
    rc = lib().oracle_accept_sample(_p(p_logits), _p(ql), V, B, L, _p(draft), T, top_p, int(top_k),
                                    int(q_mul_inv_t), int(seed) & (2**64 - 1), int(offset) & 0xFFFFFFFF,
                                    _p(n), _p(tok), _p(sl), _p(acc), _p(samp))
    assert rc == 0
    return dict(n=n, token=tok, seq_lens=sl, accept=acc[:, :L], sample=samp)


def accept_greedy(logits, draft, seq_lens=None, bf16_bits_in: bool = False):
    logits = np.ascontiguousarray(logits)
    B, W, V = logits.shape
    draft = np.ascontiguousarray(draft, dtype=np.int32).reshape(B, max(W - 1, 0))
    tt = np.zeros((B, W), np.int32)
    n = np.zeros(B, np.int32)
    tok = np.zeros(B, np.int32)
    sl = None if seq_lens is None else np.ascontiguousarray(seq_lens, dtype=np.int32).copy()
    lib().oracle_accept_greedy(_p(logits), int(bf16_bits_in), V, B, W, V, _p(draft), _p(tt), _p(n),
                               _p(tok), _p(sl))
    return dict(tt=tt, n=n, token=tok, seq_lens=sl)


def sample_rows(logits, T, top_p=1.0, top_k=0, mul_inv=False, seed=0, offset=0, row0=0):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    R, V = logits.shape
    tok = np.zeros(R, np.int32)
    pr = np.zeros((R, V), np.float32)
    lib().oracle_sample_rows(_p(logits), V, R, T, top_p, int(top_k), int(mul_inv), int(seed) & (2**64 - 1),
                             int(offset) & 0xFFFFFFFF, int(row0), _p(tok), _p(pr))
    return tok, pr


# ------------------------------------------------------------------ float64 reference algorithm
def truncate_probs_ref(p: np.ndarray, top_p: float = 1.0, top_k: int = 0) -> np.ndarray:
    """The reference's truncate_probs (src/mlx_dspark/sampling.py:18-44) in float64:
    kth-largest threshold, then the nucleus by sorted cumulative sum, then renormalise."""
    p = np.asarray(p, dtype=np.float64).copy()
    v = p.shape[-1]
    if top_p >= 1.0 and top_k <= 0:
        return p
    if 0 < top_k < v:
        kth = np.sort(p)[v - top_k]
        p = np.where(p >= kth, p, 0.0)
    if top_p < 1.0:
        sd = -np.sort(-p)
        cs = np.cumsum(sd)
        inn = (cs - sd) < top_p
        cutoff = np.min(np.where(inn, sd, np.inf))
        p = np.where(p >= cutoff, p, 0.0)
    return p / max(p.sum(), 1e-12)


def softmax64(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    e = np.exp(x - x.max())
    return e / e.sum()
