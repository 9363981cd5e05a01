"""Tensor-level wrappers over libdspark_hip.so.

Every function here launches hand-written gfx950 kernels through the C ABI on the current
torch stream; torch only provides device memory and the stream. There is no CPU path: the
tensors must live on a HIP device.
"""

from __future__ import annotations

import ctypes

import math
from dataclasses import dataclass

import torch

from . import _hip
from ._hip import (DSK_BF16, DSK_EPI_GEGLU, DSK_EPI_PARTIAL, DSK_EPI_RESIDUAL, DSK_EPI_STORE, DSK_EPI_SWIGLU, DSK_F32,
                   DSK_KV_BF16, DSK_KV_U8, call, ptr, stream_ptr)

__all__ = [
    "W8Weight", "W8Table", "Workspace", "Packed", "act_pack", "pack", "pack_rn", "w8_gemm", "w8_residual", "w8_embed",
    "w8_dequant", "rows_rmsnorm", "rows_gated",
    "qkv_rope_append", "attention", "qkv_attention", "row_logprobs", "accept_greedy", "accept_sample", "sample_rows",
    "argmax_rows", "lens_add",
    "rope_inv_freq", "DSK_EPI_STORE", "DSK_EPI_SWIGLU", "DSK_EPI_GEGLU", "DSK_EPI_PARTIAL", "DSK_KV_BF16",
    "DSK_KV_U8",
]


def _require_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("dspark kernels need device tensors (got a CPU tensor)")


# ----------------------------------------------------------------------------- workspace
class Workspace:
    """Per-device scratch for split partials and per-slice reductions.

    ``reserve`` grows a region (outside graph capture only). A captured graph keeps the raw
    address of every region it used, and a generation may widen a region after a narrower
    round was captured (a cap controller picking a wider block, a lookup round): so a region
    that is outgrown is never freed, only superseded, and every graph keeps replaying on the
    buffer it captured. Regions grow to the next power of two, which bounds the superseded
    bytes by the live ones. The kernels behind these regions hold no state between calls
    (no counters that must be zero on entry), so a fresh region needs no initialisation."""

    _per_device: dict[int, "Workspace"] = {}

    def __init__(self, device: torch.device):
        self.device = device
        self.buf: dict[str, torch.Tensor] = {}
        self.retired: list[torch.Tensor] = []

    @classmethod
    def get(cls, device) -> "Workspace":
        device = torch.device(device)
        idx = device.index if device.index is not None else torch.cuda.current_device()
        ws = cls._per_device.get(idx)
        if ws is None:
            ws = cls._per_device[idx] = Workspace(torch.device("cuda", idx))
        return ws

    def reserve(self, kind: str, nbytes: int) -> torch.Tensor:
        t = self.buf.get(kind)
        if t is not None and t.numel() >= nbytes:
            return t
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f"workspace '{kind}' must be sized before graph capture "
                               f"(need {nbytes} bytes)")
        nbytes = 1 << max(20, (int(nbytes) - 1).bit_length())
        if t is not None:
            self.retired.append(t)      # a captured graph may still replay on it
        t = torch.zeros(nbytes, dtype=torch.uint8, device=self.device)
        self.buf[kind] = t
        return t


# ----------------------------------------------------------------------------- W8 weights
@dataclass
class W8Weight:
    """An affine group-64 matrix [N, K] (8-bit codes, or 4-bit with bits=4) in the engine's tiled
    layout (see w8.hip).

    ``paired``: the rows are a gate projection stacked on an up projection, repacked so the
    GEMM's gated epilogue (SwiGLU / GeGLU) sees both halves of a column in one workgroup."""

    wt: torch.Tensor     # uint8 [N*K*bits/8]
    sb: torch.Tensor     # int32 [N/16, K/64, 16] (bf16 scale | bf16 bias << 16)
    N: int
    K: int
    paired: bool = False
    bits: int = 8

    @property
    def nbytes(self) -> int:
        return self.wt.numel() + self.sb.numel() * 4

    @staticmethod
    def quantize_mlx(w: torch.Tensor, bits: int = 8):
        """w [N, K] f32/bf16 on device -> MLX-layout codes (q u8 [N, K], 0..2^bits-1, one per
        byte), scales, biases bf16 [N, K/64]."""
        _require_cuda(w)
        if bits not in (4, 8):
            raise ValueError(f"bits={bits}: 4 or 8")
        w = w.contiguous()
        N, K = w.shape
        q = torch.empty((N, K), dtype=torch.uint8, device=w.device)
        s = torch.empty((N, K // 64), dtype=torch.bfloat16, device=w.device)
        b = torch.empty((N, K // 64), dtype=torch.bfloat16, device=w.device)
        dt = DSK_BF16 if w.dtype == torch.bfloat16 else DSK_F32
        if dt == DSK_F32 and w.dtype != torch.float32:
            w = w.float()
        call("dsk_w8_quantize" if bits == 8 else "dsk_w4_quantize", ptr(w), dt, N, K, ptr(q), ptr(s), ptr(b),
             stream_ptr())
        return q, s, b

    @classmethod
    def from_mlx(cls, q: torch.Tensor, s: torch.Tensor, b: torch.Tensor, paired: bool = False,
                 bits: int = 8) -> "W8Weight":
        """q: codes one per byte [N, K] (4-bit codes in 0..15 with bits=4)."""
        _require_cuda(q, s, b)
        N, K = q.shape
        wt = torch.empty(N * K * bits // 8, dtype=torch.uint8, device=q.device)
        sb = torch.empty((N // 16, K // 64, 16), dtype=torch.int32, device=q.device)
        call("dsk_w8_repack" if bits == 8 else "dsk_w4_repack", ptr(q.contiguous()), ptr(s.contiguous()),
             ptr(b.contiguous()), N, K, int(paired), ptr(wt), ptr(sb), stream_ptr())
        return cls(wt, sb, N, K, paired, bits)

    @classmethod
    def quantize(cls, w: torch.Tensor, paired: bool = False, bits: int = 8) -> "W8Weight":
        q, s, b = cls.quantize_mlx(w, bits)
        return cls.from_mlx(q, s, b, paired, bits)

    def rows(self, n0: int, n1: int) -> "W8Weight":
        """Zero-copy view of output rows [n0, n1) (multiples of 16, unpaired layouts)."""
        if self.paired or n0 % 16 or n1 % 16 or not 0 <= n0 < n1 <= self.N:
            raise ValueError(f"rows({n0}, {n1}) of a {self.N}-row W8 weight")
        tb = (self.K // 64) * 128 * self.bits
        return W8Weight(self.wt[n0 // 16 * tb:n1 // 16 * tb], self.sb[n0 // 16:n1 // 16], n1 - n0, self.K,
                        bits=self.bits)


@dataclass
class W8Table:
    """A W8 matrix kept in MLX row layout, for row gathers (embedding lookup)."""

    q: torch.Tensor
    s: torch.Tensor
    b: torch.Tensor

    @property
    def shape(self):
        return tuple(self.q.shape)

    def dequantize(self) -> torch.Tensor:
        V, H = self.q.shape
        w = self.q.float().view(V, H // 64, 64) * self.s.float()[..., None] + self.b.float()[..., None]
        return w.view(V, H)


# ----------------------------------------------------------------------------- GEMM path
@dataclass
class Packed:
    """An [M, K] bf16 activation in the GEMM's packed operand layout (see w8.hip).

    Normed later (``ssq`` set): the packed values are bf16(h * w) of an RMSNorm whose row scale
    rsqrt(mean(h^2) + eps) the consuming GEMM applies to its outputs; ``ssq`` f32 [M, K/16]
    holds the per-16-column partial sums of h^2 it is computed from."""

    data: torch.Tensor   # bf16, dsk_act_pack_bytes(M, K) / 2 elements
    M: int
    K: int
    ssq: torch.Tensor | None = None
    eps: float = 0.0

    @staticmethod
    def empty(M: int, K: int, device, normed_later: bool = False, eps: float = 0.0) -> "Packed":
        n = _hip.lib.dsk_act_pack_bytes(M, K)
        if n == 0:
            raise ValueError(f"cannot pack [{M}, {K}] (K must be a multiple of 64)")
        ssq = torch.empty((M, K // 16), dtype=torch.float32, device=device) if normed_later else None
        return Packed(torch.empty(n // 2, dtype=torch.bfloat16, device=device), M, K, ssq, float(eps))

    def plain(self) -> "Packed":
        """The packed values alone (a GEMM over them leaves the row scale to its consumer)."""
        return Packed(self.data, self.M, self.K)

    def row_scale(self) -> torch.Tensor | None:
        """[M] f32 rsqrt(mean(h^2) + eps) of a normed-later activation (for checks)."""
        if self.ssq is None:
            return None
        return torch.rsqrt(self.ssq.sum(1) / self.K + self.eps)

    def unpack(self) -> torch.Tensor:
        """[M, K] bf16 copy (for checks; the engine never unpacks)."""
        MT, G = (self.M + 15) // 16, self.K // 64
        v = self.data.view(MT, G, 4, 16, 16)               # [mt][g][c][r][e]
        return v.permute(0, 3, 1, 2, 4).reshape(MT * 16, self.K)[: self.M]


def _rows_ok(t: torch.Tensor) -> bool:
    return t.data_ptr() % 16 == 0 and t.stride(-1) == 1 and t.stride(0) % 8 == 0


def act_pack(*, M: int, K: int, part: torch.Tensor | None = None, h: torch.Tensor | None = None,
             copy: torch.Tensor | None = None, norm_w: torch.Tensor | None = None, eps: float = 1e-6,
             out: Packed | bool | None = True, part_norm_w: torch.Tensor | None = None,
             scale: float = 1.0) -> Packed | None:
    """Sum split-K partials [S, M, K] (f32) into the residual stream h (bf16 [M, K], in place),
    optionally copy the result (tap), RMSNorm it and pack it for the next GEMM (see
    dsk_act_pack). part_norm_w RMSNorms the partial sum before the residual add (gemma's
    sandwich norms). out=True allocates the packed output, None/False skips it."""
    if h is not None and not _rows_ok(h):
        raise ValueError("act_pack: h needs unit column stride, 16-byte aligned rows")
    if copy is not None and not _rows_ok(copy):
        raise ValueError("act_pack: copy needs unit column stride, 16-byte aligned rows")
    if part is not None and (part.dtype != torch.float32 or not part.is_contiguous() or part.shape[1:] != (M, K)):
        raise ValueError(f"act_pack: partials must be contiguous f32 [S, {M}, {K}]")
    if out is True:
        dev = (h if h is not None else part).device
        out = Packed.empty(M, K, dev)
    elif out is False:
        out = None
    call("dsk_act_pack_scaled", ptr(part), 0 if part is None else part.shape[0], ptr(part_norm_w), ptr(h),
         0 if h is None else h.stride(0),
         ptr(copy), 0 if copy is None else copy.stride(0), M, K, ptr(norm_w), float(eps), float(scale),
         ptr(None if out is None else out.data), stream_ptr())
    return out


def pack_rn(*, M: int, K: int, h: torch.Tensor, norm_w: torch.Tensor | None, eps: float,
            part: torch.Tensor | None = None, copy: torch.Tensor | None = None,
            out: Packed | None = None) -> Packed:
    """act_pack's residual add of split-K partials (or h alone), with the RMSNorm left to the
    consuming GEMM: returns the normed-later Packed bf16(h * norm_w) (dsk_act_pack_rn)."""
    if not _rows_ok(h) or (copy is not None and not _rows_ok(copy)):
        raise ValueError("pack_rn: h / copy need unit column stride, 16-byte aligned rows")
    if part is not None and (part.dtype != torch.float32 or not part.is_contiguous() or part.shape[1:] != (M, K)):
        raise ValueError(f"pack_rn: partials must be contiguous f32 [S, {M}, {K}]")
    if out is None:
        out = Packed.empty(M, K, h.device, normed_later=True, eps=eps)
    call("dsk_act_pack_rn", ptr(part), 0 if part is None else part.shape[0], ptr(h), h.stride(0), ptr(copy),
         0 if copy is None else copy.stride(0), M, K, ptr(norm_w), ptr(out.data), ptr(out.ssq), stream_ptr())
    return out


def w8_residual(x: Packed, w: W8Weight, h: torch.Tensor, *, next_norm: torch.Tensor | None, eps: float,
                copy: torch.Tensor | None = None, out: bool = True) -> Packed | None:
    """h += x . deq(W)^T in place (bf16, the residual add after o_proj / down_proj) in the
    GEMM's epilogue, copy = h (a hidden-state tap), and the next projection's input normed
    later: Packed bf16(h * next_norm) with its per-tile sums of h^2 (None when out is False)."""
    if x.K != w.K:
        raise ValueError(f"w8_residual: x has K={x.K}, W has K={w.K}")
    M = x.M
    if tuple(h.shape) != (M, w.N) or not _rows_ok(h) or (copy is not None and not _rows_ok(copy)):
        raise ValueError(f"w8_residual: h must be bf16 [{M}, {w.N}] with aligned unit-stride rows")
    y = Packed.empty(M, w.N, h.device, normed_later=True, eps=eps) if out else None
    call("dsk_w8_gemm_rn", ptr(x.data), ptr(w.wt), ptr(w.sb), w.bits, M, w.N, w.K, DSK_EPI_RESIDUAL,
         ptr(None if y is None else y.data), DSK_BF16, 0, 0.0, ptr(x.ssq), 0 if x.ssq is None else w.K // 16,
         float(x.eps), ptr(h), h.stride(0), ptr(copy), 0 if copy is None else copy.stride(0),
         ptr(next_norm if y is not None else None), ptr(None if y is None else y.ssq), stream_ptr())
    return y


def pack(x: torch.Tensor, norm_w: torch.Tensor | None = None, eps: float = 1e-6) -> Packed:
    """Pack bf16 rows x [M, K] (optionally RMSNorm-ed) for the GEMM."""
    _require_cuda(x, norm_w)
    if x.dtype != torch.bfloat16 or not _rows_ok(x):
        x = x.contiguous().to(torch.bfloat16)
    return act_pack(M=x.shape[0], K=x.shape[1], h=x, norm_w=norm_w, eps=eps)


def gemm_splits(M: int, N: int, K: int, bits: int = 8) -> int:
    """K-split slices of a DSK_EPI_PARTIAL product (the 4-bit kernel plans its own)."""
    return (_hip.lib.dsk_w8_gemm_splits if bits == 8 else _hip.lib.dsk_w4_gemm_splits)(M, N, K)


def gemm_plan(M: int, N: int, K: int, epi: int, bits: int = 8) -> tuple:
    """The plan the library runs for this GEMM: (slab_tiles, batch_groups, waves, k_splits,
    pipelined), in the terms of the explicit-plan tuning entry (dsk_w8_gemm_plan)."""
    out = (ctypes.c_int * 5)()
    call("dsk_w8_gemm_plan", int(M), int(N), int(K), int(epi), int(bits), ctypes.cast(out, ctypes.c_void_p))
    return tuple(out)


_EPILOGUE_KIND = {DSK_EPI_STORE: 0, DSK_EPI_SWIGLU: 1, DSK_EPI_GEGLU: 1, DSK_EPI_PARTIAL: 2, DSK_EPI_RESIDUAL: 3}


def gemm_kernel_name(M: int, N: int, K: int, epi: int, row_scale: bool, bits: int = 8, plan=None) -> str:
    """The kernel instantiation a GEMM launch runs (as a kernel trace names it):
    w8_gemm_kernel<row tiles, slab tiles, batch groups, waves, epilogue (+4 with the row scale
    of a normed-later x passed in), pipelined, bits>."""
    nt, u, waves, _, pf = plan or gemm_plan(M, N, K, epi, bits)
    ekr = _EPILOGUE_KIND[epi] + (4 if row_scale else 0)
    return f"w8_gemm_kernel<{(M + 15) // 16}, {nt}, {u}, {waves}, {ekr}, {'true' if pf else 'false'}, {bits}>"


def w8_gemm(x: Packed, w: W8Weight, *, epi: int = DSK_EPI_STORE, out=None, out_dtype: torch.dtype = torch.bfloat16,
            residual: torch.Tensor | None = None, softcap: float = 0.0):
    """x . deq(W)^T for a packed x (M <= 64). Returns, by epilogue:
    STORE   -> [M, N] (out_dtype; + residual; soft-cap)
    PARTIAL -> f32 [S, M, N] split-K partial sums (S = gemm_splits(M, N, K))
    SWIGLU / GEGLU (paired W) -> Packed [M, N/2], the next GEMM's x."""
    M = x.M
    if x.K != w.K:
        raise ValueError(f"w8_gemm: x has K={x.K}, W has K={w.K}")
    dev = x.data.device
    ldy, yd = 0, DSK_BF16
    if epi == DSK_EPI_STORE:
        if out is None:
            out = torch.empty((M, w.N), dtype=out_dtype, device=dev)
        ydata, ldy, yd = out, out.stride(0), (DSK_F32 if out.dtype == torch.float32 else DSK_BF16)
    elif epi == DSK_EPI_PARTIAL:
        S = gemm_splits(M, w.N, w.K, w.bits)
        if out is None:
            out = torch.empty((S, M, w.N), dtype=torch.float32, device=dev)
        elif tuple(out.shape) != (S, M, w.N) or out.dtype != torch.float32:
            raise ValueError(f"w8_gemm: partial output must be f32 [{S}, {M}, {w.N}]")
        ydata, yd = out, DSK_F32
    else:
        if not w.paired:
            raise ValueError("gated epilogue needs a paired gate|up weight")
        if out is None:
            out = Packed.empty(M, w.N // 2, dev)
        ydata = out.data
    if x.ssq is not None:
        if residual is not None:
            raise ValueError("w8_gemm: a normed-later x takes no residual (use w8_residual)")
        call("dsk_w8_gemm_rn", ptr(x.data), ptr(w.wt), ptr(w.sb), w.bits, M, w.N, w.K, int(epi), ptr(ydata), yd, ldy,
             float(softcap), ptr(x.ssq), w.K // 16, float(x.eps), None, 0, None, 0, None, None, stream_ptr())
        return out
    call("dsk_w8_gemm" if w.bits == 8 else "dsk_w4_gemm", ptr(x.data), ptr(w.wt), ptr(w.sb), M, w.N, w.K, int(epi),
         ptr(ydata), yd, ldy, ptr(residual), residual.stride(0) if residual is not None else 0, float(softcap),
         stream_ptr())
    return out


def w8_dequant(w: W8Weight, out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16 [N, K] rows bf16(s * q + b) of a W8 / W4 weight in source row order (a paired
    gate|up weight: the gate rows, then the up rows), for a library GEMM over many rows."""
    n = w.N * w.K
    if out is None:
        out = torch.empty((w.N, w.K), dtype=torch.bfloat16, device=w.wt.device)
    elif out.dtype != torch.bfloat16 or not out.is_contiguous() or out.numel() < n:
        raise ValueError("w8_dequant: out must be a contiguous bf16 buffer of N*K elements")
    out = out.view(-1)[:n].view(w.N, w.K)
    call("dsk_w8_dequant_rows", ptr(w.wt), ptr(w.sb), w.bits, w.N, w.K, int(w.paired), ptr(out), stream_ptr())
    return out


def rows_rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16((x * rsqrt(mean(x^2) + eps)) * w) over the rows of x [M, K] bf16 (any M)."""
    if x.dtype != torch.bfloat16 or not _rows_ok(x):
        raise ValueError("rows_rmsnorm: x must be bf16 with unit column stride and aligned rows")
    out = torch.empty_like(x) if out is None else out
    call("dsk_rows_rmsnorm", ptr(x), x.stride(0), ptr(w), float(eps), x.shape[0], x.shape[1], ptr(out), out.stride(0),
         stream_ptr())
    return out


def rows_gated(gu: torch.Tensor, act: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16(bf16(act(gate)) * up) for gu [M, 2I] bf16 = [gate | up] rows (act = DSK_EPI_SWIGLU
    or DSK_EPI_GEGLU), as the GEMM's gated epilogue."""
    M, I2 = gu.shape
    out = torch.empty((M, I2 // 2), dtype=torch.bfloat16, device=gu.device) if out is None else out
    call("dsk_rows_gated", ptr(gu), gu.stride(0), M, I2 // 2, int(act), ptr(out), out.stride(0), stream_ptr())
    return out


def w8_embed(ids: torch.Tensor, table: W8Table, scale: float = 1.0, out: torch.Tensor | None = None):
    ids = ids.reshape(-1)
    if ids.dtype != torch.int32:
        ids = ids.to(torch.int32)
    V, H = table.q.shape
    n = ids.numel()
    if out is None:
        out = torch.empty((n, H), dtype=torch.bfloat16, device=ids.device)
    call("dsk_w8_embed", ptr(ids), n, ptr(table.q), ptr(table.s), ptr(table.b), V, H, float(scale),
         ptr(out), out.stride(0), stream_ptr())
    return out


# ----------------------------------------------------------------------------- attention
def rope_inv_freq(head_dim: int, theta: float, device, *, rotary_fraction: float = 1.0) -> torch.Tensor:
    """theta ** (-2 d / head_dim) for d < head_dim / 2, computed in float64, stored f32.
    rotary_fraction < 1 is proportional RoPE (gemma4): only the first
    int(rotary_fraction * head_dim / 2) frequencies rotate, with exponents still over the full
    head_dim; the rest are 0 (those dims pass through)."""
    d = torch.arange(0, head_dim // 2, dtype=torch.float64)
    inv = theta ** (-2.0 * d / head_dim)
    if rotary_fraction < 1.0:
        inv[int(rotary_fraction * head_dim // 2):] = 0.0
    return inv.to(torch.float32).to(device)


def qkv_rope_append(qkv, B, W, nq, nkv, hd, q_norm, k_norm, eps, inv_freq, seq_lens, block_table,
                    page, kv_dtype, k_pool, v_pool, k_sb=None, v_sb=None, q_out=None, pos_offset=0, v_norm=None,
                    x: Packed | None = None):
    """qkv: bf16 [B*W, (nq+2nkv)*hd] or f32 split-K partials [S, B*W, (nq+2nkv)*hd]. v_norm
    (bf16 [hd]) RMSNorms V too. x: the projection's normed-later input, whose row scale the
    summed partials take here (the projection then ran without it)."""
    splits = qkv.shape[0] if qkv.dim() == 3 else 0
    if splits and (qkv.dtype != torch.float32 or not qkv.is_contiguous()):
        raise ValueError("qkv partials must be contiguous f32")
    if not splits and (qkv.dtype != torch.bfloat16 or not qkv.is_contiguous()):
        qkv = qkv.contiguous().to(torch.bfloat16)
    if q_out is None and nq:
        q_out = torch.empty((B * W, nq * hd), dtype=torch.bfloat16, device=qkv.device)
    if x is not None and x.ssq is not None:
        if pos_offset or v_norm is not None:
            raise ValueError("qkv_rope_append: a normed-later input takes no pos_offset / v_norm")
        call("dsk_qkv_rope_append_rn", ptr(qkv), splits, B, W, nq, nkv, hd, ptr(q_norm), ptr(k_norm), float(eps),
             ptr(inv_freq), ptr(seq_lens), ptr(block_table), block_table.shape[1], page, kv_dtype, ptr(k_pool),
             ptr(v_pool), ptr(k_sb), ptr(v_sb), ptr(q_out), ptr(x.ssq), x.K // 16, float(x.eps), stream_ptr())
        return q_out
    call("dsk_qkv_norm_rope_append", ptr(qkv), splits, B, W, nq, nkv, hd, ptr(q_norm), ptr(k_norm), ptr(v_norm),
         float(eps), ptr(inv_freq), ptr(seq_lens), int(pos_offset), ptr(block_table), block_table.shape[1], page,
         kv_dtype, ptr(k_pool), ptr(v_pool), ptr(k_sb), ptr(v_sb), ptr(q_out), stream_ptr())
    return q_out


def attention(q, B, W, nq, nkv, hd, scale, seq_lens, max_ctx, block_table, page, kv_dtype, k_pool,
              v_pool, k_sb=None, v_sb=None, *, causal=True, window=0, softcap=0.0, out=None, packed=False):
    """Returns bf16 [B*W, nq*hd], or a Packed [B*W, nq*hd] (the o-projection's x) when packed."""
    if out is None:
        out = Packed.empty(B * W, nq * hd, q.device) if packed else torch.empty(
            (B * W, nq * hd), dtype=torch.bfloat16, device=q.device)
    odata = out.data if isinstance(out, Packed) else out
    ws = Workspace.get(q.device)
    need = _hip.lib.dsk_attn_ws_bytes(B, W, nq, hd, max_ctx)
    buf = ws.reserve("attn", need)
    call("dsk_attention", ptr(q), B, W, nq, nkv, hd, float(scale), int(bool(causal)), int(window),
         float(softcap), ptr(seq_lens), int(max_ctx), ptr(block_table), block_table.shape[1], page,
         kv_dtype, ptr(k_pool), ptr(v_pool), ptr(k_sb), ptr(v_sb), ptr(odata), int(isinstance(out, Packed)),
         ptr(buf), buf.numel(), stream_ptr())
    return out



def qkv_attention(qkv, B, W, nq, nkv, hd, q_norm, k_norm, eps, inv_freq, scale, seq_lens, max_ctx, block_table,
                  page, kv_dtype, k_pool, v_pool, k_sb=None, v_sb=None, *, causal=True, window=0, softcap=0.0,
                  out=None, packed=False):
    """qkv_rope_append + attention in one kernel: qkv is the projection (bf16 [B*W, (nq+2nkv)*hd]
    or f32 split-K partials [S, B*W, (nq+2nkv)*hd]); the W new tokens' K/V are appended to the
    pool at seq_lens[b] + i. Returns bf16 [B*W, nq*hd] or a Packed when packed."""
    splits = qkv.shape[0] if qkv.dim() == 3 else 0
    if splits and (qkv.dtype != torch.float32 or not qkv.is_contiguous()):
        raise ValueError("qkv partials must be contiguous f32")
    if not splits and (qkv.dtype != torch.bfloat16 or not qkv.is_contiguous()):
        qkv = qkv.contiguous().to(torch.bfloat16)
    if out is None:
        out = Packed.empty(B * W, nq * hd, qkv.device) if packed else torch.empty(
            (B * W, nq * hd), dtype=torch.bfloat16, device=qkv.device)
    odata = out.data if isinstance(out, Packed) else out
    ws = Workspace.get(qkv.device)
    buf = ws.reserve("attn", _hip.lib.dsk_attn_ws_bytes(B, W, nq, hd, max_ctx))
    call("dsk_qkv_attention", ptr(qkv), splits, B, W, nq, nkv, hd, ptr(q_norm), ptr(k_norm), float(eps),
         ptr(inv_freq), float(scale), int(bool(causal)), int(window), float(softcap), ptr(seq_lens), int(max_ctx),
         ptr(block_table), block_table.shape[1], page, kv_dtype, ptr(k_pool), ptr(v_pool), ptr(k_sb), ptr(v_sb),
         ptr(odata), int(isinstance(out, Packed)), ptr(buf), buf.numel(), stream_ptr())
    return out

# ----------------------------------------------------------------------------- acceptance
def accept_greedy(logits: torch.Tensor, draft: torch.Tensor | None, *, seq_lens=None, tt=None,
                  n_out=None, token_out=None):
    """logits [B, W, V] (f32/bf16), draft [B, W-1] int32 -> (tt [B, W], n [B], token [B])."""
    B, W, V = logits.shape
    dev = logits.device
    if logits.stride(2) != 1 or logits.stride(1) != V or logits.stride(0) != W * V:
        logits = logits.contiguous()
    tt = torch.empty((B, W), dtype=torch.int32, device=dev) if tt is None else tt
    n_out = torch.empty(B, dtype=torch.int32, device=dev) if n_out is None else n_out
    token_out = torch.empty(B, dtype=torch.int32, device=dev) if token_out is None else token_out
    dt = DSK_BF16 if logits.dtype == torch.bfloat16 else DSK_F32
    ws = Workspace.get(dev)
    need = _hip.lib.dsk_accept_ws_bytes(B, W, V)
    buf = ws.reserve("accept", need)
    call("dsk_accept_greedy", ptr(logits), dt, V, B, W, V, ptr(draft), ptr(tt), ptr(n_out), ptr(token_out),
         ptr(seq_lens), ptr(buf), buf.numel(), stream_ptr())
    return tt, n_out, token_out


def accept_sample(p_logits: torch.Tensor, q_logits: torch.Tensor | None, draft: torch.Tensor,
                  temperature: float, top_p: float = 1.0, top_k: int = 0, *, q_mul_inv_t: bool = False,
                  seed: int = 0, offset: int = 0, seq_lens=None, n_out=None, token_out=None,
                  accept_out=None, sample_out=None, offset_dev=None):
    """p_logits [B, L+1, V] f32, q_logits [B, L, V] f32 or None (one-hot q), draft [B, L] int32."""
    B, R, V = p_logits.shape
    L = R - 1
    dev = p_logits.device
    p_logits = p_logits.contiguous().float()
    if q_logits is not None:
        q_logits = q_logits.contiguous().float()
    n_out = torch.empty(B, dtype=torch.int32, device=dev) if n_out is None else n_out
    token_out = torch.empty(B, dtype=torch.int32, device=dev) if token_out is None else token_out
    ws = Workspace.get(dev)
    need = _hip.lib.dsk_accept_ws_bytes(B, R, V)
    buf = ws.reserve("accept", need)
    call("dsk_accept_sample", ptr(p_logits), ptr(q_logits), V, B, L, ptr(draft), float(temperature),
         float(top_p), int(top_k or 0), int(bool(q_mul_inv_t)), int(seed) & ((1 << 64) - 1),
         int(offset) & 0xFFFFFFFF, ptr(n_out), ptr(token_out), ptr(seq_lens), ptr(accept_out),
         ptr(sample_out), ptr(buf), buf.numel(), ptr(offset_dev), stream_ptr())
    return n_out, token_out


def sample_rows(logits: torch.Tensor, temperature: float, top_p: float = 1.0, top_k: int = 0, *,
                mul_inv_t: bool = False, seed: int = 0, offset: int = 0, row0: int = 0,
                token_out=None, probs_out=None, offset_dev=None):
    """logits [R, V] f32 -> tokens [R] (argmax at temperature 0) and, when probs_out [R, V] f32 is
    given, the truncated distribution each row was drawn from."""
    R, V = logits.shape
    if temperature <= 0 and R <= 1024 and logits.dtype in (torch.float32, torch.bfloat16):
        return argmax_rows(logits, token_out=token_out), probs_out
    logits = logits.contiguous().float()
    token_out = torch.empty(R, dtype=torch.int32, device=logits.device) if token_out is None else token_out
    buf = Workspace.get(logits.device).reserve("sample", _hip.lib.dsk_sample_ws_bytes(R, V))
    call("dsk_sample_rows", ptr(logits), V, R, float(temperature), float(top_p), int(top_k or 0),
         int(bool(mul_inv_t)), int(seed) & ((1 << 64) - 1), int(offset) & 0xFFFFFFFF, int(row0),
         ptr(token_out), ptr(probs_out), ptr(offset_dev), ptr(buf), buf.numel(), stream_ptr())
    return token_out, probs_out


def argmax_rows(logits: torch.Tensor, *, token_out=None) -> torch.Tensor:
    """logits [R, V] f32/bf16 (rows may be strided) -> argmax per row, int32 [R] (lowest index on
    ties), each row split over 64 workgroups."""
    R, V = logits.shape
    if logits.stride(1) != 1 or logits.stride(0) < V:
        logits = logits.contiguous()
    token_out = torch.empty(R, dtype=torch.int32, device=logits.device) if token_out is None else token_out
    dt = DSK_BF16 if logits.dtype == torch.bfloat16 else DSK_F32
    buf = Workspace.get(logits.device).reserve("argmax", _hip.lib.dsk_argmax_ws_bytes(R))
    call("dsk_argmax_rows", ptr(logits), dt, logits.stride(0), V, R, ptr(token_out), ptr(buf), buf.numel(),
         stream_ptr())
    return token_out


def prefetch(w: W8Weight, sink: torch.Tensor, workgroups: int = 512) -> None:
    """Read a weight's codes and scale words on the current stream and keep nothing
    (dsk_prefetch): run on a side stream, it brings them into the memory-side cache for the
    GEMM that reads them next. sink: a 16-byte device buffer the kernel may write."""
    for t in (w.wt, w.sb):
        call("dsk_prefetch", ptr(t), t.numel() * t.element_size(), int(workgroups), ptr(sink), stream_ptr())


def lens_add(lens: torch.Tensor, n: torch.Tensor | None, add: int) -> None:
    call("dsk_lens_add", ptr(lens), ptr(n), lens.numel(), int(add), stream_ptr())


# ----------------------------------------------------------------------------- DSpark Markov head
MARKOV_MAX_B = 16  # batch rows of one dsk_markov_block call


def markov_block(base_logits: torch.Tensor, first_prev: torch.Tensor, w1: W8Table, w2: W8Weight, *,
                 temperature: float = 0.0, top_p: float = 1.0, top_k: int = 0, seed: int = 0, offset: int = 0,
                 tok_out: torch.Tensor | None = None, q_logits_out: torch.Tensor | None = None):
    """Sequential block sampling with the rank-R Markov head (see markov.hip).

    base_logits f32 [B, cap, V] (or [cap, V]), first_prev int32 [B] on device. Greedy
    (temperature 0) -> tokens int32 [B, cap]; sampled -> (tokens, q_logits [B, cap, V]), the
    step logits whose truncated softmax at 1/T each token was drawn from."""
    if base_logits.dim() == 2:
        base_logits = base_logits.unsqueeze(0)
    B, cap, V = base_logits.shape
    if base_logits.dtype != torch.float32 or base_logits.stride(2) != 1 or base_logits.stride(1) != base_logits.stride(2) * V \
            or base_logits.stride(0) != cap * V:
        base_logits = base_logits.float().contiguous()
    dev = base_logits.device
    first_prev = first_prev.reshape(-1)
    if first_prev.dtype != torch.int32:
        first_prev = first_prev.to(torch.int32)
    tok_out = torch.empty((B, cap), dtype=torch.int32, device=dev) if tok_out is None else tok_out
    sampled = temperature > 0
    if sampled and q_logits_out is None:
        q_logits_out = torch.empty((B, cap, V), dtype=torch.float32, device=dev)
    R = w1.q.shape[1]
    ws = Workspace.get(dev)
    # pieces of MARKOV_MAX_B rows (the kernel's tile); row0 keeps every row's Philox stream
    for b0 in range(0, B, MARKOV_MAX_B):
        b1 = min(B, b0 + MARKOV_MAX_B)
        buf = ws.reserve("markov", _hip.lib.dsk_markov_ws_bytes(b1 - b0, V, int(sampled)))
        call("dsk_markov_block", ptr(base_logits[b0:b1]), V, b1 - b0, cap, V, R, ptr(first_prev[b0:b1]), ptr(w1.q),
             ptr(w1.s), ptr(w1.b), ptr(w2.wt), ptr(w2.sb), float(temperature), float(top_p), int(top_k or 0),
             int(seed) & ((1 << 64) - 1), int(offset) & 0xFFFFFFFF, b0, ptr(tok_out[b0:b1]),
             ptr(q_logits_out[b0:b1] if sampled else None), ptr(buf), buf.numel(), stream_ptr())
    return (tok_out, q_logits_out) if sampled else tok_out


def logits_penalize(logits: torch.Tensor, row_ptr: torch.Tensor, ids: torch.Tensor, vals: torch.Tensor) -> None:
    """logits[r, ids[j]] -= vals[j] for j in [row_ptr[r], row_ptr[r+1]) (CSR rows, in place)."""
    R = logits.shape[0]
    call("dsk_logits_penalize", ptr(logits), logits.stride(0), R, ptr(row_ptr), ptr(ids), ptr(vals), stream_ptr())


# ----------------------------------------------------------------------------- logprobs
def row_logprobs(logits: torch.Tensor, tokens: torch.Tensor, top_k: int = 0):
    """logits [R, V] f32 (unit column stride), tokens int32 [R] -> (chosen f32 [R], top_ids
    int32 [R, top_k], top_vals f32 [R, top_k]) of log_softmax(logits) (see dsk_row_logprobs)."""
    R, V = logits.shape
    if logits.dtype != torch.float32 or logits.stride(1) != 1:
        logits = logits.float().contiguous()
    dev = logits.device
    tokens = tokens.to(dev, torch.int32).contiguous()
    chosen = torch.empty(R, dtype=torch.float32, device=dev)
    ids = torch.empty((R, max(top_k, 1)), dtype=torch.int32, device=dev)
    vals = torch.empty((R, max(top_k, 1)), dtype=torch.float32, device=dev)
    call("dsk_row_logprobs", ptr(logits), logits.stride(0), R, V, ptr(tokens), int(top_k), ptr(chosen), ptr(ids),
         ptr(vals), stream_ptr())
    return chosen, ids[:, :top_k], vals[:, :top_k]
