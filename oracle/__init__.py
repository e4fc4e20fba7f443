"""CPU oracle for the axk hot path — TEST INFRASTRUCTURE ONLY.

A restatement, in numpy / torch-CPU fp32 (and plain C for the MXFP4 codec, oracle/mx_codec.c), of the
reference algorithms of ZHEQIUSHUI/ax-dsl-kernels for the per-layer Qwen3.5 hot path. Each function
cites the reference file:line it follows. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this package, and only as the checker or the timed CPU baseline — the
product path (ax-dsl-kernels_amd/axk) never calls it.

Pinning status of each module is recorded in its own header.
"""
