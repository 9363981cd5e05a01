"""CPU oracle for the MI355X speculative-decoding verify engine.

TEST INFRASTRUCTURE ONLY: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg may import this package, and only as the checker (or the timed CPU baseline). The
engine (mlx-dspark_amd/mlx_dspark) never imports it and has no CPU fallback.

Contents (each function cites the reference file:line it restates):
  accept.py  -- acceptance / sampling (C restatement in accept_oracle.c, ctypes wrapper)
  w8.py      -- W8 affine group-64 quantize / dequantize / GEMM (numpy)
  model.py   -- Qwen3-shaped verify forward with hidden-state tap, paged-KV semantics,
                DSpark and DFlash drafter forwards (torch on the CPU, float32)

Pinning (what checks each function against something other than itself) is listed in each
module's header; anything without such a check is marked "parity unpinned" there.
"""
