"""Benchmark of the axk hot path on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Prints ONE JSON line (rank 0) with the BASELINE metric for the chosen workload, the roofline of its
dominant kernel and a CPU baseline (the oracle timed on the host cores over a bounded sample).
Inputs are synthetic (seeded), resident in HBM before the timed region; weight / KV buffers rotate over
>= 1 GiB of distinct copies so the 256 MB MALL cannot serve them.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "ax-dsl-kernels_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFS = 2500.0  # dense MFMA peaks of MI355X: bf16, fp8, fp4 (the prefill kernels' MFMAs are bf16, fp32 acc)
FP8_PEAK_TFS = 5000.0
FP4_PEAK_TFS = 10100.0


def mfma_fracs(tflops: float) -> dict:
    """Achieved TFLOP/s as fractions of the dense bf16, fp8 and fp4 MFMA peaks."""
    return {"bf16_mfma_frac": round(tflops / BF16_PEAK_TFS, 4), "fp8_mfma_frac": round(tflops / FP8_PEAK_TFS, 4),
            "fp4_mfma_frac": round(tflops / FP4_PEAK_TFS, 4)}


def tokens_per_s(wl, ms_per_step: float):
    """Tokens per second through the path: the step's tokens over its time (None for a workload without tokens)."""
    return round(wl.tokens / (ms_per_step * 1e-3), 1) if wl.tokens else None
ROTATE_BYTES = 1 << 30
METRIC = "µs/decode-layer + achieved HBM GB/s (% of 8 TB/s) for MXFP4 MoE + paged attn"


def _cpu_threads() -> int:
    """Threads the CPU baseline uses: the CPUs this process may run on, at most 16 (the GPU box's CPU share)."""
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count() or 1
    return max(1, min(16, avail))


def cpu_machine() -> dict:
    """The host the CPU baseline ran on: CPU model, logical CPUs, physical cores and the CPUs this process may use."""
    model, phys = None, set()
    cur = {}
    try:
        with open("/proc/cpuinfo", encoding="utf-8") as f:
            for ln in f:
                if ":" not in ln:
                    if "core id" in cur:
                        phys.add((cur.get("physical id", "0"), cur["core id"]))
                    cur = {}
                    continue
                k, v = (x.strip() for x in ln.split(":", 1))
                cur[k] = v
                if k == "model name" and model is None:
                    model = v
        if "core id" in cur:
            phys.add((cur.get("physical id", "0"), cur["core id"]))
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = None
    return {"cpu_model": model, "logical_cpus": os.cpu_count(), "physical_cores": len(phys) or None,
            "cpus_available": affinity}


def _time_cpu(fn, budget_s: float = 10.0, min_reps: int = 3, max_reps: int = 50) -> tuple[float, int]:
    """Median seconds per call of fn over a bounded number of repetitions (~budget_s of CPU work)."""
    fn()  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < max_reps and (len(times) < min_reps or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


class Workload:
    """A step is pre() + main() + post(); the roofline kernel is launched by main()."""

    in_suite = True
    traffic_profile = None  # profiles/ file holding the kernel's measured HBM bytes per launch
    tokens = None  # tokens one step carries through the path (decode: one per sequence; prefill: the chunk)

    def pre(self, i: int) -> None:
        pass

    def main(self, i: int) -> None:
        self.step(i)

    def post(self, i: int) -> None:
        pass


class MxLinearWorkload(Workload):
    """Config 0: one MXFP4 linear, W 4096 x 4096 (E2M1 + E8M0), x bf16 [1, 4096], bf16 out."""

    name = "mxfp4_linear"
    tokens = 1  # tokens one step carries through the path
    kernel = "mx_group_kernel"
    timing = "graph"
    traffic_profile = "mxfp4_linear_config0_pmc.txt"

    def __init__(self, dev):
        import torch

        from axk import configs

        c = configs.config0()
        self.host = c
        self.m, self.n, self.k = 1, 4096, 4096
        # algorithmic bytes per launch: codes + scales + x + out
        self.alg_bytes = self.n * self.k // 2 + self.n * self.k // 32 + 2 * self.m * self.k + 2 * self.m * self.n
        self.alg_flops = 2 * self.m * self.n * self.k
        per_copy = self.n * self.k // 2 + self.n * self.k // 32
        self.copies = max(2, -(-ROTATE_BYTES // per_copy))
        w, s = c["w"].to(dev), c["s"].to(dev)
        self.w = [w.clone() for _ in range(self.copies)]
        self.s = [s.clone() for _ in range(self.copies)]
        self.x = c["x"].to(dev)
        self.out = torch.empty(self.m, self.n, dtype=torch.bfloat16, device=dev)
        self.config = {"workload": "config0: MXFP4 linear N=4096 K=4096 M=1", "rotating_copies": self.copies}
        self.dtype = "mxfp4 x bf16 -> fp32 acc"

    def step(self, i: int) -> None:
        import axk

        j = i % self.copies
        axk.mxfp4_gemm(self.x, self.w[j], self.s[j], output=self.out)

    def cpu_baseline(self) -> dict:
        from oracle import _c

        x = self.host["x"].view(__import__("torch").int16).numpy().view("u2")
        w, s = self.host["w"].numpy(), self.host["s"].numpy()
        nt = _cpu_threads()
        sec, reps = _time_cpu(lambda: _c.mxfp4_linear(x, w, s, nthreads=nt))
        return {"value": sec * 1e6, "unit": "µs/op", "cores": nt, "kind": "port",
                "sample": f"full config0 op (oracle/mx_codec.c, OpenMP), median of {reps} runs"}


class MxLinearPrefillWorkload(Workload):
    """Config 0's MXFP4 weight (4096 x 4096) at prefill rows: x bf16 [4096, 4096], bf16 out: the dense GEMM path of
    axk_mxfp4_gemm (m >= 128). MFMA-bound: 2 M N K flops against dense bf16 (the weights are decoded exactly to bf16
    in registers, the activations are bf16)."""

    name = "mxfp4_linear_prefill"
    tokens = 4096  # tokens one step carries through the path
    kernel = "mx_gemm_kernel<0, 0>"
    timing = "graph"
    mfma = True
    traffic_profile = "mxfp4_linear_prefill_m4096_pmc.txt"

    def __init__(self, dev):
        import torch

        from axk import configs

        c = configs.config0()
        g = torch.Generator().manual_seed(1)
        self.m, self.n, self.k = 4096, 4096, 4096
        self.host = (torch.randn(self.m, self.k, generator=g).to(torch.bfloat16), c["w"], c["s"])
        self.alg_bytes = self.n * self.k // 2 + self.n * self.k // 32 + 2 * self.m * self.k + 2 * self.m * self.n
        self.alg_flops = 2 * self.m * self.n * self.k
        w, s = c["w"].to(dev), c["s"].to(dev)
        # the activations (32 MiB) and outputs rotate with the weights so the MALL serves no repeated bytes
        per_copy = self.alg_bytes
        self.copies = max(2, -(-ROTATE_BYTES // per_copy))
        self.x = [self.host[0].to(dev) for _ in range(self.copies)]
        self.w = [w.clone() for _ in range(self.copies)]
        self.s = [s.clone() for _ in range(self.copies)]
        self.out = [torch.empty(self.m, self.n, dtype=torch.bfloat16, device=dev) for _ in range(self.copies)]
        self.config = {"workload": "MXFP4 linear N=4096 K=4096 at M=4096 prefill rows (config 0's weight)",
                       "rotating_copies": self.copies}
        self.dtype = "mxfp4 x bf16 -> fp32 acc"

    def step(self, i: int) -> None:
        import axk

        j = i % self.copies
        axk.mxfp4_gemm(self.x[j], self.w[j], self.s[j], output=self.out[j])

    def cpu_baseline(self) -> dict:
        import torch

        from oracle import _c

        x, w, s = self.host
        rows = 64  # a bounded sample of the 4096 rows, scaled by rows
        xs = x[:rows].contiguous().view(torch.int16).numpy().view("u2")
        nt = _cpu_threads()
        sec, reps = _time_cpu(lambda: _c.mxfp4_linear(xs, w.numpy(), s.numpy(), nthreads=nt), budget_s=10.0,
                              min_reps=1, max_reps=5)
        return {"value": sec * self.m / rows * 1e6, "unit": "µs/op", "cores": nt, "kind": "port",
                "sample": f"{rows} of the {self.m} rows (oracle/mx_codec.c, OpenMP), scaled by rows, median of "
                          f"{reps} runs"}


class LmHeadWorkload(Workload):
    """The MXFP4 LM head GEMV of decode (a row next to the path): W [248320, 2048] (E2M1 + E8M0, config 0's encoding),
    x bf16 [1, 2048], fp32 logits (mul_mat_mx4_n248320_k2048, q35_layer_mc.py:705-724)."""

    name = "lm_head"
    tokens = 1  # tokens one step carries through the path
    kernel = "mx_group_kernel<0, 1, 4, 0, 4>"
    timing = "graph"
    traffic_profile = "lm_head_vocab248320_pmc.txt"

    def __init__(self, dev):
        import torch

        from axk import configs

        self.m, self.n, self.k = 1, configs.LM_HEAD["vocab"], configs.LM_HEAD["hidden"]
        per_copy = self.n * self.k // 2 + self.n * self.k // 32
        # algorithmic bytes per launch: codes + scales + x + fp32 logits
        self.alg_bytes = per_copy + 2 * self.m * self.k + 4 * self.m * self.n
        self.alg_flops = 2 * self.m * self.n * self.k
        self.copies = max(2, -(-ROTATE_BYTES // per_copy))
        c = [configs.lm_head_case(dev, seed=i) for i in range(self.copies)]
        self.w, self.s, self.x = [ci["w"] for ci in c], [ci["s"] for ci in c], c[0]["x"]
        self.out = torch.empty(self.m, self.n, dtype=torch.float32, device=dev)
        self.config = {"workload": f"MXFP4 LM head GEMV N={self.n} K={self.k} M=1, fp32 logits",
                       "rotating_copies": self.copies}
        self.dtype = "mxfp4 x bf16 -> fp32 acc"

    def step(self, i: int) -> None:
        import torch

        import axk

        j = i % self.copies
        axk.mxfp4_gemm(self.x, self.w[j], self.s[j], out_dtype=torch.float32, output=self.out)

    def cpu_baseline(self) -> dict:
        from oracle import _c

        rows = 16384  # a bounded sample of the vocabulary's rows, scaled to the whole head
        x = self.x.cpu().view(__import__("torch").int16).numpy().view("u2")
        w, s = self.w[0][:rows].cpu().numpy(), self.s[0][:rows].cpu().numpy()
        nt = _cpu_threads()
        sec, reps = _time_cpu(lambda: _c.mxfp4_linear(x, w, s, nthreads=nt))
        return {"value": sec * 1e6 * self.n / rows, "unit": "µs/op", "cores": nt, "kind": "port",
                "sample": f"{rows} of the {self.n} rows (oracle/mx_codec.c, OpenMP), median of {reps} runs, "
                          f"scaled by rows"}


class LmHeadNvfp4Workload(Workload):
    """The LM head in NVFP4 (the reference's NVFP4 head, test_nvfp4_lm_head.py; nvfp4_gemm, gemm.py:495-561):
    W [248320, 2048] E2M1 pairs with E4M3 scales per 16 along K and an fp32 scale2, x bf16 [1, 2048], fp32 logits.
    Each code is decoded at scale 1 and multiplied by its block's E4M3 scale in fp32 (gfx950's scaled converts take
    only a power of two), so the decode costs more VALU than the MXFP4 head's."""

    name = "lm_head_nvfp4"
    tokens = 1  # tokens one step carries through the path
    kernel = "mx_group_kernel<5, 1, 4, 0, 4>"
    timing = "graph"
    traffic_profile = "lm_head_nvfp4_vocab248320_pmc.txt"

    def __init__(self, dev):
        import torch

        from axk import configs

        self.m, self.n, self.k = 1, configs.LM_HEAD["vocab"], configs.LM_HEAD["hidden"]
        per_copy = self.n * self.k // 2 + self.n * self.k // 16
        # algorithmic bytes per launch: codes + E4M3 scales + scale2 + x + fp32 logits
        self.alg_bytes = per_copy + 4 + 2 * self.m * self.k + 4 * self.m * self.n
        self.alg_flops = 2 * self.m * self.n * self.k
        self.copies = max(2, -(-ROTATE_BYTES // per_copy))
        c = [configs.lm_head_nvfp4_case(dev, seed=i) for i in range(self.copies)]
        self.w, self.s, self.s2, self.x = [ci["w"] for ci in c], [ci["s"] for ci in c], c[0]["s2"], c[0]["x"]
        self.out = torch.empty(self.m, self.n, dtype=torch.float32, device=dev)
        self.config = {"workload": f"NVFP4 LM head GEMV N={self.n} K={self.k} M=1, fp32 logits",
                       "rotating_copies": self.copies}
        self.dtype = "nvfp4 x bf16 -> fp32 acc"

    def step(self, i: int) -> None:
        import torch

        import axk

        j = i % self.copies
        axk.nvfp4_gemm(self.x, self.w[j], self.s[j], self.s2, out_dtype=torch.float32, output=self.out)

    def cpu_baseline(self) -> dict:
        import torch

        from oracle import mx

        rows = 4096  # a bounded sample of the vocabulary's rows, scaled to the whole head
        x = self.x.cpu()
        w, s, s2 = self.w[0][:rows].cpu().numpy(), self.s[0][:rows].cpu().numpy(), self.s2.item()
        nt = _cpu_threads()
        torch.set_num_threads(nt)
        sec, reps = _time_cpu(lambda: mx.nvfp4_linear(x, w, s, s2))
        return {"value": sec * 1e6 * self.n / rows, "unit": "µs/op", "cores": nt, "kind": "port",
                "sample": f"{rows} of the {self.n} rows (oracle/mx.py: numpy dequant + torch fp32 matmul), median of "
                          f"{reps} runs, scaled by rows"}


class PagedDecodeWorkload(Workload):
    """Config 1: paged decode attention, batch 16, 16 q / 2 KV heads, D 256, page 64, L_b ~ U[1024, 16384].

    One step = plan (split-KV partition) + split (the attention kernel) + merge (LSE merge of split partials),
    captured with the other steps in one HIP graph (as a serving decode step is).
    The roofline is the split kernel's: algorithmic bytes = K and V rows of every valid token + q + out +
    page table.
    """

    name = "paged_decode"
    tokens = 16  # tokens one step carries through the path
    kernel = "paged_decode_kernel<256, 2, 0>"  # launched by axk_paged_decode_split
    timing = "graph"       # value: K steps (plan + split + merge) replayed as one HIP graph
    traffic_profile = "paged_decode_config1_pmc.txt"

    def __init__(self, dev):
        import torch

        from axk import attention, configs

        c = configs.config1()
        self.host = c
        self.lens = c["lens"]
        tot = sum(self.lens)
        b, hq, d = c["q"].shape
        hkv = c["cache"].shape[3]
        npages = int(c["indptr"][-1])
        self.alg_bytes = tot * 2 * hkv * d * 2 + 2 * b * hq * d * 2 + 4 * (npages + 2 * b + 1)
        self.alg_flops = 4 * tot * hq * d
        per_copy = c["cache"].numel() * 2
        self.copies = max(2, -(-ROTATE_BYTES // per_copy))
        cache = c["cache"].to(dev)
        self.caches = [cache] + [cache.clone() for _ in range(self.copies - 1)]
        self.q = c["q"].to(dev)
        self.indptr, self.indices, self.last = (c[k].to(dev) for k in ("indptr", "indices", "last_page_len"))
        self.out = torch.empty_like(self.q)
        self.ws = attention.paged_decode_workspace(b, hq, hkv, d, dev)
        from axk import _lib

        lib = _lib.load()
        self._plan = lambda: lib.axk_paged_decode_plan(self.indptr.data_ptr(), self.last.data_ptr(), b, hq, hkv, d,
                                                       c["cache"].shape[2], self.ws.data_ptr(), self.ws.numel(),
                                                       torch.cuda.current_stream().cuda_stream)
        self._split = lambda cache: lib.axk_paged_decode_split(
            self.q.data_ptr(), cache.data_ptr(), self.indptr.data_ptr(), self.indices.data_ptr(),
            self.last.data_ptr(), self.out.data_ptr(), b, hq, hkv, d, c["cache"].shape[2], c["cache"].shape[0],
            c["scale"], self.ws.data_ptr(), self.ws.numel(), torch.cuda.current_stream().cuda_stream)
        self._merge = lambda: lib.axk_paged_decode_merge(self.indptr.data_ptr(), self.last.data_ptr(),
                                                         self.out.data_ptr(), b, hq, hkv, d, c["cache"].shape[2],
                                                         self.ws.data_ptr(), self.ws.numel(),
                                                         torch.cuda.current_stream().cuda_stream)
        self.config = {"workload": "config1: paged decode B=16 HQ=16 HKV=2 D=256 page=64 L~U[1024,16384]",
                       "sum_context": tot, "rotating_copies": self.copies}
        self.dtype = "bf16 (fp32 softmax / accumulation)"

    def pre(self, i: int) -> None:
        assert self._plan() == 0

    def main(self, i: int) -> None:
        assert self._split(self.caches[i % self.copies]) == 0

    def post(self, i: int) -> None:
        assert self._merge() == 0

    def step(self, i: int) -> None:
        self.pre(i)
        self.main(i)
        self.post(i)

    def roofline_step(self, i: int) -> None:
        """The split kernel alone (the plan and the merge are other launches)."""
        self.main(i)

    def cpu_baseline(self) -> dict:
        import torch

        from oracle import paged_attn

        c = self.host
        nt = _cpu_threads()
        torch.set_num_threads(nt)
        sec, reps = _time_cpu(lambda: paged_attn.paged_decode(c["q"], c["cache"], c["indptr"], c["indices"],
                                                              c["last_page_len"], c["scale"]), budget_s=10.0,
                              min_reps=2, max_reps=10)
        return {"value": sec * 1e6, "unit": "µs/op", "cores": nt, "kind": "port",
                "sample": f"full config1 op (oracle/paged_attn.py, torch fp32 CPU), median of {reps} runs"}


def encode_cache(cache, dev, kind: str, kv_scale: float = 1.0):
    """A bf16 paged cache [P, 2, page, HKV, D] written whole through the product's KV write kernels (every (page, slot)
    row as one cache_location): the FP8 cache's codes, or the INT8 cache's (codes, scales)."""
    import torch

    from axk import attention

    p, _, page, hkv, d = cache.shape
    rows = p * page
    k = cache[:, 0].reshape(rows, hkv, d).contiguous().to(dev)
    v = cache[:, 1].reshape(rows, hkv, d).contiguous().to(dev)
    loc = torch.stack([torch.arange(p).repeat_interleave(page), torch.arange(page).repeat(p)], 1)
    loc = loc.to(torch.int32).contiguous().to(dev)
    if kind == "fp8":
        codes = torch.zeros(p, 2, page, hkv, d, dtype=torch.uint8, device=dev)
        attention.store_paged_kv_fp8(k, v, codes, loc, kv_scale)
        return codes
    codes = torch.zeros(p, 2, page, hkv, d, dtype=torch.int8, device=dev)
    scales = torch.zeros(p, 2, page, hkv, dtype=torch.bfloat16, device=dev)
    attention.store_paged_kv_i8(k, v, codes, scales, loc)
    return codes, scales


class PagedDecodeFp8Workload(Workload):
    """Config 1's attention over an FP8 E4M3 cache (the FP8 cache, KV8 = 2, q35_group.py:44-54): the same
    sequences, pages and queries, the cache stored as e4m3(bf16(x * 8)). One step = axk_paged_decode_fp8 (plan +
    split + merge); the roofline is the whole op's (so it includes the merge): K and V bytes of every valid token
    (half of bf16's) + q + out + page table."""

    name = "paged_decode_fp8kv"
    tokens = 16  # tokens one step carries through the path
    kernel = "paged_decode_kernel<256, 1> (+ merge)"
    timing = "graph"
    traffic_profile = "paged_decode_fp8kv_config1_pmc.txt"  # every kernel of the op, summed
    KV_SCALE = 8.0

    def __init__(self, dev):
        import torch

        from axk import attention, configs

        c = configs.config1()
        self.host = c
        tot = sum(c["lens"])
        b, hq, d = c["q"].shape
        pool, _, page, hkv, _ = c["cache"].shape
        npages = int(c["indptr"][-1])
        self.alg_bytes = tot * 2 * hkv * d + 2 * b * hq * d * 2 + 4 * (npages + 2 * b + 1)
        self.alg_flops = 4 * tot * hq * d
        codes = encode_cache(c["cache"], dev, "fp8", self.KV_SCALE)
        self.copies = max(2, -(-ROTATE_BYTES // codes.numel()))
        self.caches = [codes] + [codes.clone() for _ in range(self.copies - 1)]
        self.q = c["q"].to(dev)
        self.indptr, self.indices, self.last = (c[k].to(dev) for k in ("indptr", "indices", "last_page_len"))
        self.out = torch.empty_like(self.q)
        self.ws = attention.paged_decode_workspace(b, hq, hkv, d, dev)
        self.scale = c["scale"]
        self.config = {"workload": "config1 over an FP8 E4M3 KV cache (kv_scale 8): B=16 HQ=16 HKV=2 D=256 page=64",
                       "sum_context": tot, "rotating_copies": self.copies}
        self.dtype = "fp8 e4m3 KV -> bf16 (fp32 softmax / accumulation)"

    def step(self, i: int) -> None:
        import axk

        axk.paged_decode_fp8(self.q, self.caches[i % self.copies], self.indptr, self.indices, self.last,
                             self.KV_SCALE, sm_scale=self.scale, output=self.out, workspace=self.ws)

    def cpu_baseline(self) -> dict:
        import torch

        from oracle import paged_attn

        c = self.host
        deq = paged_attn.dequant_kv_fp8(paged_attn.quant_kv_fp8(c["cache"], self.KV_SCALE), self.KV_SCALE)
        nt = _cpu_threads()
        torch.set_num_threads(nt)
        sec, reps = _time_cpu(lambda: paged_attn.paged_decode(c["q"], deq, c["indptr"], c["indices"],
                                                              c["last_page_len"], c["scale"]), budget_s=10.0,
                              min_reps=2, max_reps=10)
        return {"value": sec * 1e6, "unit": "µs/op", "cores": nt, "kind": "port",
                "sample": f"full config1 op on the dequantised FP8 cache (oracle/paged_attn.py, torch fp32 CPU), "
                          f"median of {reps} runs"}


class PagedDecodeI8Workload(PagedDecodeFp8Workload):
    """Config 1's attention over an INT8 cache (the INT8 cache, KV8 = 1, q35_group.py:44-47, 197-221): the same
    sequences, pages and queries, each row and KV head stored as int8 codes with a bf16 scale. One step =
    axk_paged_decode_i8 (plan + split + merge); algorithmic bytes: the codes and scales of every valid token + q + out
    + page table."""

    name = "paged_decode_i8kv"
    tokens = 16  # tokens one step carries through the path
    kernel = "paged_decode_kernel<256, 1, 1> (+ merge)"
    traffic_profile = "paged_decode_i8kv_config1_pmc.txt"  # every kernel of the op, summed

    def __init__(self, dev):
        import torch

        from axk import attention, configs

        c = configs.config1()
        self.host = c
        tot = sum(c["lens"])
        b, hq, d = c["q"].shape
        pool, _, page, hkv, _ = c["cache"].shape
        npages = int(c["indptr"][-1])
        self.alg_bytes = tot * 2 * hkv * (d + 2) + 2 * b * hq * d * 2 + 4 * (npages + 2 * b + 1)
        self.alg_flops = 4 * tot * hq * d
        codes, scales = encode_cache(c["cache"], dev, "i8")
        self.copies = max(2, -(-ROTATE_BYTES // codes.numel()))
        self.caches = [(codes, scales)] + [(codes.clone(), scales.clone()) for _ in range(self.copies - 1)]
        self.q = c["q"].to(dev)
        self.indptr, self.indices, self.last = (c[k].to(dev) for k in ("indptr", "indices", "last_page_len"))
        self.out = torch.empty_like(self.q)
        self.ws = attention.paged_decode_workspace(b, hq, hkv, d, dev)
        self.scale = c["scale"]
        self.config = {"workload": "config1 over an INT8 KV cache (bf16 scale per row and KV head): B=16 HQ=16 HKV=2 "
                                   "D=256 page=64", "sum_context": tot, "rotating_copies": self.copies}
        self.dtype = "int8 KV + bf16 row scales -> bf16 (fp32 softmax / accumulation)"

    def step(self, i: int) -> None:
        import axk

        codes, scales = self.caches[i % self.copies]
        axk.paged_decode_i8(self.q, codes, scales, self.indptr, self.indices, self.last, sm_scale=self.scale,
                            output=self.out, workspace=self.ws)

    def cpu_baseline(self) -> dict:
        import torch

        from oracle import paged_attn

        c = self.host
        deq = paged_attn.dequant_kv_i8(*paged_attn.quant_kv_i8(c["cache"]))
        nt = _cpu_threads()
        torch.set_num_threads(nt)
        sec, reps = _time_cpu(lambda: paged_attn.paged_decode(c["q"], deq, c["indptr"], c["indices"],
                                                              c["last_page_len"], c["scale"]), budget_s=10.0,
                              min_reps=2, max_reps=10)
        return {"value": sec * 1e6, "unit": "µs/op", "cores": nt, "kind": "port",
                "sample": f"full config1 op on the dequantised INT8 cache (oracle/paged_attn.py, torch fp32 CPU), "
                          f"median of {reps} runs"}


class PagedPrefillWorkload(Workload):
    """Prefill attention (G x P-row causal block attention, q35_prefill.py:264-336; flash_attn.py:
    471-611): one sequence's 4096-token chunk over an empty history in the paged cache, config 1's attention shape
    (HQ 16 / HKV 2, D 256, page 64). One step = axk_paged_prefill (one launch). MFMA-bound: the flops of the visible
    (query, key) pairs only, 4 D HQ sum_t (t + 1) (QK^T and PV), against dense bf16."""

    name = "paged_prefill"
    tokens = 4096  # tokens one step carries through the path
    kernel = "paged_prefill_kernel<256>"
    timing = "graph"
    mfma = True
    traffic_profile = "paged_prefill_chunk4096_pmc.txt"
    T = 4096

    def __init__(self, dev):
        import torch

        from axk import configs

        g = torch.Generator().manual_seed(0)
        c = configs.prefill_case([self.T], [self.T], 16, 2, 256, 64, g)
        self.host = c
        self.d = {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in c.items()}
        hq, d = 16, 256
        self.alg_flops = 4 * d * hq * (self.T * (self.T + 1) // 2)
        self.alg_bytes = 2 * c["q"].numel() * 2 + c["cache"].numel() * 2 + 4 * (c["indices"].numel() + 4)
        self.out = torch.empty_like(self.d["q"])
        self.config = {"workload": "prefill chunk: B=1, T=4096 new tokens, empty history, HQ=16 HKV=2 D=256 page=64, "
                                   "causal"}
        self.dtype = "bf16 (fp32 softmax / accumulation)"

    def step(self, i: int) -> None:
        from axk import attention

        d = self.d
        attention.paged_prefill(d["q"], d["cache"], d["qo_indptr"], d["indptr"], d["indices"], d["last_page_len"],
                                sm_scale=self.host["scale"], output=self.out)

    def cpu_baseline(self) -> dict:
        import torch

        from oracle import paged_attn

        c = self.host
        nt = _cpu_threads()
        torch.set_num_threads(nt)
        sec, reps = _time_cpu(lambda: paged_attn.paged_prefill(c["q"], c["cache"], c["qo_indptr"], c["indptr"],
                                                               c["indices"], c["last_page_len"], c["scale"]),
                              budget_s=10.0, min_reps=1, max_reps=5)
        return {"value": sec * 1e6, "unit": "µs/op", "cores": nt, "kind": "port",
                "sample": f"the full 4096-token chunk (oracle/paged_attn.py paged_prefill, torch fp32 CPU), "
                          f"median of {reps} runs"}


class GdnDecodeWorkload(Workload):
    """Config 2 decode: GDN recurrent step, B = 32, 32 value / 16 key heads, d = 128, fp32 state in place."""

    name = "gdn_decode"
    tokens = 32  # tokens one step carries through the path
    kernel = "gdn_recurrent_kernel<false>"
    timing = "graph"
    traffic_profile = "gdn_decode_config2a_pmc.txt"

    def __init__(self, dev):
        import torch

        from axk import configs

        c = configs.config2_decode()
        self.host = c
        self.d = {k: v.to(dev) for k, v in c.items()}
        st = c["state"]
        # algorithmic bytes: state read + write, q, k, v, out, a, b
        self.alg_bytes = 2 * st.numel() * 4 + 2 * (c["q"].numel() + c["k"].numel() + 2 * c["v"].numel()) + \
            2 * (c["a"].numel() + c["b"].numel())
        self.copies = max(2, -(-ROTATE_BYTES // (st.numel() * 4)))
        self.states = [self.d["state"].clone() for _ in range(self.copies)]
        self.out = torch.empty_like(self.d["v"])
        self.config = {"workload": "config2a: GDN decode B=32 NV=32 NK=16 d=128 (state in place)",
                       "rotating_copies": self.copies}
        self.dtype = "fp32 state, bf16 io"

    def step(self, i: int) -> None:
        from axk import gdn

        d = self.d
        s = self.states[i % self.copies]
        gdn.gdn_recurrent(d["q"], d["k"], d["v"], d["a"], d["b"], d["a_log"], d["dt_bias"], s, state_out=s,
                          output=self.out)

    def cpu_baseline(self) -> dict:
        import torch

        from oracle import gdn as ogdn

        c = self.host
        nt = _cpu_threads()
        torch.set_num_threads(nt)
        sec, reps = _time_cpu(lambda: ogdn.gdn_fp32(c["q"], c["k"], c["v"], c["a"], c["b"], c["a_log"],
                                                     c["dt_bias"], c["state"]), budget_s=10.0, min_reps=2,
                              max_reps=20)
        return {"value": sec * 1e6, "unit": "µs/op", "cores": nt, "kind": "port",
                "sample": f"full config2a step (oracle/gdn.py gdn_fp32, torch CPU), median of {reps} runs"}


class GdnPrefillWorkload(Workload):
    """Config 2 prefill: GDN chunked prefill, B = 1, T = 4096, chunk 64, 32 value / 16 key heads, zero state.

    One step = the chunk-parallel solve kernel + the state-scan kernel. Algorithmic bytes: q, k, v, a, b in,
    output out, fp32 state in and out; algorithmic flops: the chunked form's products per (head, chunk)."""

    name = "gdn_prefill"
    tokens = 4096  # tokens one step carries through the path
    kernel = "gdn chunk step (prep + scan)"
    timing = "graph"
    mfma = True
    traffic_profile = "gdn_prefill_config2b_pmc.txt"

    def __init__(self, dev):
        import torch

        from axk import configs, gdn

        c = configs.config2_prefill()
        self.host = c
        self.d = {k: v.to(dev) for k, v in c.items()}
        b, t, nk, dk = c["q"].shape
        nv = c["v"].shape[2]
        st = c["state"]
        self.alg_bytes = 2 * (c["q"].numel() + c["k"].numel() + 2 * c["v"].numel() + c["a"].numel() +
                              c["b"].numel()) + 2 * st.numel() * 4
        chunks = -(-t // 64)
        per = 2 * 64 * 64 * dk * 5 + 2 * 64 * dk * dk * 3  # K K^T, Q K^T, u, w, P v_new; w S, q S, k^T X
        self.alg_flops = b * nv * chunks * per
        self.ws = gdn.gdn_chunk_workspace(b, t, nk, nv, dev)
        self.state_out = torch.empty_like(self.d["state"])
        self.out = torch.empty_like(self.d["v"])
        self.config = {"workload": "config2b: GDN chunked prefill B=1 T=4096 C=64 NV=32 NK=16 d=128 (zero state)"}
        self.dtype = "bf16 operands, fp32 accumulation / state"

    def step(self, i: int) -> None:
        from axk import gdn

        d = self.d
        gdn.gdn_chunk_prefill(d["q"], d["k"], d["v"], d["a"], d["b"], d["a_log"], d["dt_bias"], d["state"],
                              state_out=self.state_out, output=self.out, workspace=self.ws)

    def cpu_baseline(self) -> dict:
        import torch

        from oracle import gdn as ogdn

        c = self.host
        nt = _cpu_threads()
        torch.set_num_threads(nt)
        sec, reps = _time_cpu(lambda: ogdn.gdn_chunk(c["q"], c["k"], c["v"], c["a"], c["b"], c["a_log"],
                                                      c["dt_bias"], c["state"], chunk=64, round_bf16=False),
                              budget_s=10.0, min_reps=1, max_reps=5)
        return {"value": sec * 1e6, "unit": "µs/op", "cores": nt, "kind": "port",
                "sample": f"full config2b prefill (oracle/gdn.py gdn_chunk fp32, torch CPU), median of {reps} runs"}


class MoeDecodeWorkload(Workload):
    """Config 3a: MoE layer decode, 32 tokens, hidden 2048, 256 MXFP4 experts (inter 512) + shared, top-8.

    One step = router GEMV + top-K + grouping + gate-up/SwiGLU + down + combine (6 launches, one graph).
    Algorithmic bytes: the weights of the experts actually routed (U distinct) + shared expert + router +
    activations in/out."""

    name = "moe_decode"
    tokens = 32  # tokens one step carries through the path
    kernel = "moe step (router, route, group, gateup, down, combine)"
    timing = "graph"
    traffic_profile = "moe_decode_config3a_pmc.txt"

    def __init__(self, dev):
        import torch

        from axk import configs, moe

        c = configs.config3(32)
        self.host = c
        w = c["weights"]
        per_expert = sum(w[n][0].numel() for n in ("e_gw", "e_gs", "e_dw", "e_ds"))
        shared = sum(w[n].numel() for n in ("w_gate", "s_gate", "w_up", "s_up", "w_down", "s_down"))
        expert_bytes = per_expert * w["e_gw"].shape[0]
        self.copies = max(2, -(-ROTATE_BYTES // expert_bytes))
        wd = {n: v.to(dev) for n, v in w.items()}
        self.wsets = [wd] + [{n: (v.clone() if n.startswith("e_") else v) for n, v in wd.items()}
                             for _ in range(self.copies - 1)]
        self.h2, self.x = c["h2"].to(dev), c["x_res"].to(dev)
        self.out = torch.empty_like(self.h2)
        self.ws = moe.moe_workspace(32, 2048, 256, 8, 512, 512, dev)
        _, _, ids, _ = moe.moe_decode(self.h2, wd, top_k=8, x_res=self.x, output=self.out, workspace=self.ws)
        self.active = int(torch.unique(ids).numel())
        self.alg_bytes = self.active * per_expert + shared + w["w_router"].numel() * 2 + w["w_shg"].numel() * 2 + \
            3 * self.h2.numel() * 2
        self.config = {"workload": "config3a: MoE decode T=32 H=2048 E=256 F=512 top-8 + shared (MXFP4)",
                       "distinct_experts": self.active, "rotating_copies": self.copies}
        self.dtype = "mxfp4 weights x bf16 -> fp32 acc"

    def step(self, i: int) -> None:
        from axk import moe

        moe.moe_decode(self.h2, self.wsets[i % self.copies], top_k=8, x_res=self.x, output=self.out,
                       workspace=self.ws)

    def cpu_baseline(self) -> dict:
        import torch

        from oracle import moe as omoe

        c = self.host
        nt = _cpu_threads()
        torch.set_num_threads(nt)
        sec, reps = _time_cpu(lambda: omoe.moe_layer(c["h2"], c["weights"], 8, x_res=c["x_res"]), budget_s=10.0,
                              min_reps=1, max_reps=5)
        return {"value": sec * 1e6, "unit": "µs/op", "cores": nt, "kind": "port",
                "sample": f"full config3a layer (oracle/moe.py, numpy dequant + torch CPU), median of {reps} runs"}


class MoeLayerDecodeWorkload(Workload):
    """The 35B's MoE decode layer (gdn_layer_full_mx, q35_layer_mc.py:855-866): a GDN layer (16 key / 32 value heads,
    hidden 2048, MXFP8 projections) whose MLP is the MoE block (shared expert MXFP8 inter 512, 256 MXFP4 experts of
    512, top-8), 32 sequences as config 3a, state and conv state in place.

    One step = the layer's 7 launches before the MLP, the shared expert's two, and config 3a's routed path, one graph.
    Algorithmic bytes: every weight of the layer and the shared expert, the router, the routed experts actually
    used (U distinct), the fp32 state read and written, the conv state, activations in and out."""

    name = "moe_layer_decode"
    tokens = 32  # tokens one step carries through the path
    kernel = "35B MoE decode layer (GDN half + shared expert + routed experts)"
    timing = "graph"
    traffic_profile = "moe_layer_decode_b32_pmc.txt"  # every kernel of the step, summed

    def __init__(self, dev):
        import torch

        from axk import configs, layer

        self.b, self.h, self.nk, self.nv = 32, 2048, 16, 32
        g = torch.Generator().manual_seed(0)
        w = configs.gdn_layer_weights(g, self.h, 512, self.nk, self.nv, proj_fmt="mxfp8", mlp_fmt="mxfp8")
        blk = configs.moe_block(g, self.h, 256, 512, 8)
        x = torch.randn(self.b, self.h, generator=g).bfloat16()
        st = torch.randn(self.b, self.nv, 128, 128, generator=g) * 0.02
        cv = torch.randn(self.b, 3, 2 * self.nk * 128 + self.nv * 128, generator=g).bfloat16()
        self.host = (w, blk, x, st, cv)
        per_expert = sum(blk[n][0].numel() for n in ("e_gw", "e_gs", "e_dw", "e_ds"))
        layer_bytes = sum(v.numel() * v.element_size() for v in w.values())
        set_bytes = layer_bytes + per_expert * 256
        self.copies = max(2, -(-ROTATE_BYTES // set_bytes))
        wd = {n: v.to(dev) for n, v in w.items()}
        bd = {n: (v.to(dev) if torch.is_tensor(v) else v) for n, v in blk.items()}
        self.wsets = [(wd, bd)] + [({n: v.clone() for n, v in wd.items()},
                                    {n: (v.clone() if torch.is_tensor(v) else v) for n, v in bd.items()})
                                   for _ in range(self.copies - 1)]
        self.scopies = max(2, -(-ROTATE_BYTES // (st.numel() * 4)))
        self.states = [st.to(dev) for _ in range(self.scopies)]
        self.convs = [cv.to(dev) for _ in range(self.scopies)]
        self.x = x.to(dev)
        self.out = torch.empty_like(self.x)
        self.ws = layer.gdn_workspace(self.b, self.h, self.nk, self.nv, 512, dev, moe=bd)
        ids = torch.empty(self.b, 8, dtype=torch.int32, device=dev)
        layer.gdn_layer_decode(self.x, wd, self.states[0].clone(), self.convs[0].clone(), self.nk, self.nv,
                               workspace=self.ws, proj_fmt="mxfp8", mlp_fmt="mxfp8",
                               moe=dict(bd, topk_ids=ids))
        self.active = int(torch.unique(ids).numel())
        self.alg_bytes = layer_bytes + blk["w_router"].numel() * 2 + blk["w_shg"].numel() * 2 + \
            self.active * per_expert + 2 * st.numel() * 4 + 2 * cv.numel() * 2 + 2 * x.numel() * 2
        self.config = {"workload": "35B MoE decode layer: GDN (16/32 heads, H=2048, MXFP8) + MoE (shared MXFP8 "
                                   "F=512, 256 MXFP4 experts F=512, top-8), B=32",
                       "distinct_experts": self.active, "rotating_copies": self.copies}
        self.dtype = "mxfp8 / mxfp4 weights x bf16 -> fp32 acc, fp32 state"

    def step(self, i: int) -> None:
        from axk import layer

        wd, bd = self.wsets[i % self.copies]
        s, c = self.states[i % self.scopies], self.convs[i % self.scopies]
        layer.gdn_layer_decode(self.x, wd, s, c, self.nk, self.nv, workspace=self.ws, out=self.out, state_out=s,
                               conv_out=c, proj_fmt="mxfp8", mlp_fmt="mxfp8", moe=bd)

    def cpu_baseline(self) -> dict:
        import torch

        from oracle import layer as olayer

        w, blk, x, st, cv = self.host
        nt = _cpu_threads()
        torch.set_num_threads(nt)
        n = 4  # a bounded sample: 4 of the 32 sequences, scaled by sequences

        def run():
            y, _, _ = olayer.gdn_layer_half(x[:n], w, st[:n], cv[:n], self.nk, self.nv, proj_fmt="mxfp8")
            return olayer.moe_block_parts(x[:n], y, w, blk, fmt="mxfp8")

        sec, reps = _time_cpu(run, budget_s=10.0, min_reps=1, max_reps=3)
        return {"value": sec * self.b / n * 1e6, "unit": "µs/op", "cores": nt, "kind": "port",
                "sample": f"oracle/layer.py on {n} of the {self.b} sequences (GDN half + MoE block), scaled by "
                          f"sequences, median of {reps} runs"}


class MoeLayerPrefillWorkload(Workload):
    """The 35B's MoE prefill layer (qwen35moe_gdn_prefill, q35_moe_prefill.py:47-52, then its routed experts and
    combine 150-214): a prompt chunk of 4096 tokens through a GDN layer (16 key / 32 value heads, hidden 2048, MXFP8
    projections) whose MLP is the MoE block (shared expert MXFP8 inter 512, 256 MXFP4 experts of 512, top-8), state
    and conv state in place.

    One step = the layer's launches (rmsnorm, the qkv | z | b | a GEMMs, conv, chunk prep + scan, gated norm, the
    output GEMM), the shared expert's two GEMMs and config 3b's routed path, one graph. Algorithmic flops: every
    projection, the shared and routed experts, the router and the chunked delta rule's products; bytes: the weights
    (every expert is routed at this size), the state read and written, activations in and out."""

    name = "moe_layer_prefill"
    tokens = 4096  # tokens one step carries through the path
    kernel = "35B MoE prefill layer (GDN prefill + shared expert + grouped routed experts)"
    timing = "graph"
    mfma = True
    traffic_profile = "moe_layer_prefill_t4096_pmc.txt"  # every kernel of the step, summed

    def __init__(self, dev):
        import torch

        from axk import configs, layer

        self.t, self.h, self.nk, self.nv, e, fe, k = 4096, 2048, 16, 32, 256, 512, 8
        g = torch.Generator().manual_seed(0)
        w = configs.gdn_layer_weights(g, self.h, 512, self.nk, self.nv, proj_fmt="mxfp8", mlp_fmt="mxfp8")
        blk = configs.moe_block(g, self.h, e, fe, k)
        x = torch.randn(1, self.t, self.h, generator=g).bfloat16()
        st = torch.randn(1, self.nv, 128, 128, generator=g) * 0.02
        cv = torch.randn(1, 3, 2 * self.nk * 128 + self.nv * 128, generator=g).bfloat16()
        self.host = (w, blk, x, st, cv)
        self.wd = {n: v.to(dev) for n, v in w.items()}
        self.bd = {n: (v.to(dev) if torch.is_tensor(v) else v) for n, v in blk.items()}
        self.x, self.st, self.cv = x.to(dev), st.to(dev), cv.to(dev)
        self.out = torch.empty_like(self.x)
        self.ws = layer.gdn_prefill_workspace(1, self.t, self.h, self.nk, self.nv, 512, dev, moe=self.bd)
        per_expert = sum(blk[n][0].numel() for n in ("e_gw", "e_gs", "e_dw", "e_ds"))
        layer_bytes = sum(v.numel() * v.element_size() for v in w.values())
        r, hh, kd, vd = self.t, self.h, self.nk * 128, self.nv * 128
        c = 2 * kd + vd
        self.alg_bytes = layer_bytes + blk["w_router"].numel() * 2 + blk["w_shg"].numel() * 2 + e * per_expert + \
            2 * st.numel() * 4 + 2 * cv.numel() * 2 + 2 * x.numel() * 2
        proj = 2 * r * hh * (c + vd + 2 * self.nv) + 2 * r * vd * hh
        shared = 2 * r * hh * 2 * 512 + 2 * r * 512 * hh
        routed = r * k * (2 * hh * 2 * fe + 2 * fe * hh)
        chunk = self.nv * (-(-r // 64)) * (2 * 64 * 64 * 128 * 5 + 2 * 64 * 128 * 128 * 3)
        self.alg_flops = proj + shared + routed + 2 * r * hh * e + chunk
        self.config = {"workload": "35B MoE prefill layer: GDN (16/32 heads, H=2048, MXFP8) + MoE (shared MXFP8 "
                                   "F=512, 256 MXFP4 experts F=512, top-8), B=1, T=4096"}
        self.dtype = "mxfp8 / mxfp4 weights x bf16 -> fp32 acc, fp32 state"

    def step(self, i: int) -> None:
        from axk import layer

        layer.gdn_layer_prefill(self.x, self.wd, self.st, self.cv, self.nk, self.nv, workspace=self.ws, out=self.out,
                                state_out=self.st, conv_out=self.cv, proj_fmt="mxfp8", mlp_fmt="mxfp8", moe=self.bd)

    def cpu_baseline(self) -> dict:
        import torch

        from oracle import layer as olayer

        w, blk, x, st, cv = self.host
        nt = _cpu_threads()
        torch.set_num_threads(nt)
        n = 128  # a bounded sample: the first 128 tokens, scaled by tokens

        def run():
            y, _, _, _ = olayer.gdn_prefill_half(x[:, :n], w, st, cv, self.nk, self.nv, proj_fmt="mxfp8")
            return olayer.moe_block_parts(x[0, :n], y, w, blk, fmt="mxfp8")

        sec, reps = _time_cpu(run, budget_s=10.0, min_reps=1, max_reps=3)
        return {"value": sec * self.t / n * 1e6, "unit": "µs/op", "cores": nt, "kind": "port",
                "sample": f"oracle/layer.py on the first {n} of the {self.t} tokens (GDN prefill half + MoE block), "
                          f"scaled by tokens, median of {reps} runs"}


class CopyCalibWorkload(Workload):
    """A plain 256 MiB device-to-device copy: the known-size kernel that calibrates the FETCH_SIZE /
    WRITE_SIZE counters (read 256 MiB, write 256 MiB per launch)."""

    name = "copy_calib"
    kernel = "__amd_rocclr_copyBuffer"
    timing = "events"
    in_suite = False

    def __init__(self, dev):
        import torch

        self.n = 256 << 20
        self.src = torch.randint(0, 255, (self.n,), dtype=torch.uint8, device=dev)
        self.dst = torch.empty_like(self.src)
        self.alg_bytes = 2 * self.n
        self.config = {"workload": "copy calibration: 256 MiB device-to-device"}
        self.dtype = "u8"

    def step(self, i: int) -> None:
        self.dst.copy_(self.src)

    def cpu_baseline(self) -> dict:
        return None


class MoePrefillWorkload(Workload):
    """Config 3b: MoE layer prefill, 4096 tokens, hidden 2048, 256 MXFP4 experts (inter 512) + shared, top-8.

    One step = router GEMM + top-K + blocked grouping + grouped gate-up/SwiGLU and down GEMMs (MFMA, bf16
    operands from in-register MXFP4 decode) + combine. Algorithmic bytes: every expert's weights (all are routed
    at this size), shared expert, router, activations in / residual in / out; flops: router, routed and shared
    experts."""

    name = "moe_prefill"
    tokens = 4096  # tokens one step carries through the path
    kernel = "moe prefill step"
    timing = "graph"
    mfma = True
    traffic_profile = "moe_prefill_config3b_pmc.txt"

    def __init__(self, dev):
        import torch

        from axk import configs, moe

        t = 4096
        c = configs.config3(t)
        w = c["weights"]
        e, two_f, hh = w["e_gw"].shape
        hidden, inter = 2 * hh, two_f // 2
        per_expert = sum(w[n][0].numel() for n in ("e_gw", "e_gs", "e_dw", "e_ds"))
        shared = sum(w[n].numel() for n in ("w_gate", "s_gate", "w_up", "s_up", "w_down", "s_down"))
        self.wd = {n: v.to(dev) for n, v in w.items()}
        self.h2, self.x = c["h2"].to(dev), c["x_res"].to(dev)
        self.out = torch.empty_like(self.h2)
        self.ws = moe.moe_workspace(t, hidden, e, 8, inter, inter, dev)
        self.alg_bytes = e * per_expert + shared + w["w_router"].numel() * 2 + 3 * t * hidden * 2
        per_row = 2 * hidden * 2 * inter + 2 * inter * hidden  # gate-up + down of one (token, expert)
        self.alg_flops = t * 8 * per_row + t * per_row + 2 * t * hidden * e
        self.config = {"workload": "config3b: MoE prefill T=4096 H=2048 E=256 F=512 top-8 + shared (MXFP4)"}
        self.dtype = "mxfp4 weights x bf16 -> fp32 acc"

    def step(self, i: int) -> None:
        from axk import moe

        moe.moe_decode(self.h2, self.wd, top_k=8, x_res=self.x, output=self.out, workspace=self.ws)

    def cpu_baseline(self) -> dict:
        import torch

        from axk import configs
        from oracle import moe as omoe

        sample = 256  # tokens of the 4096 (same weights), scaled to the full step
        c = configs.config3(4096)
        h2, x = c["h2"][:sample], c["x_res"][:sample]
        nt = _cpu_threads()
        torch.set_num_threads(nt)
        sec, reps = _time_cpu(lambda: omoe.moe_layer(h2, c["weights"], 8, x_res=x), budget_s=10.0, min_reps=1,
                              max_reps=5)
        return {"value": sec * 1e6 * (4096 / sample), "unit": "µs/op", "cores": nt, "kind": "port",
                "sample": f"{sample} of the 4096 config3b tokens (oracle/moe.py moe_layer, torch CPU), median of "
                          f"{reps} runs, scaled x{4096 // sample} to the full step"}


class MxDequantWorkload(Workload):
    """Config 0's weight through the standalone codec: E2M1 codes + E8M0 scales -> exact fp32 [4096, 4096].

    Algorithmic bytes: codes + scales read, fp32 values written."""

    name = "mxfp4_dequant"
    kernel = "mxfp4_dequant_kernel"
    timing = "graph"
    traffic_profile = "mxfp4_dequant_config0_pmc.txt"

    def __init__(self, dev):
        import torch

        from axk import configs

        c = configs.config0()
        self.host = c
        n, k = 4096, 4096
        self.alg_bytes = n * k // 2 + n * k // 32 + 4 * n * k
        per_copy = n * k // 2 + n * k // 32
        self.copies = max(2, -(-ROTATE_BYTES // (per_copy + 4 * n * k)))
        w, s = c["w"].to(dev), c["s"].to(dev)
        self.w = [w.clone() for _ in range(self.copies)]
        self.s = [s.clone() for _ in range(self.copies)]
        self.out = [torch.empty(n, k, dtype=torch.float32, device=dev) for _ in range(self.copies)]
        self.config = {"workload": "config0 weight: MXFP4 dequant N=4096 K=4096 -> fp32", "rotating_copies": self.copies}
        self.dtype = "u8 codes / E8M0 -> f32"

    def step(self, i: int) -> None:
        import axk

        j = i % self.copies
        axk.mxfp4_dequant(self.w[j], self.s[j], output=self.out[j])

    def cpu_baseline(self) -> dict:
        from oracle import _c

        w, s = self.host["w"].numpy(), self.host["s"].numpy()
        sec, reps = _time_cpu(lambda: _c.mxfp4_dequant(w, s))
        return {"value": sec * 1e6, "unit": "µs/op", "cores": 1, "kind": "port",
                "sample": f"full config0 weight (oracle/mx_codec.c, one thread), median of {reps} runs"}


class Fp8LinearWorkload(Workload):
    """Config 4's largest FP8 projection: E4M3 weight [16384, 4096] + f32 per-channel scale, x bf16 [8, 4096]
    (the group's decode batch), bf16 out. Algorithmic bytes: weight + scales + x + out."""

    name = "fp8_linear"
    tokens = 8  # tokens one step carries through the path
    kernel = "mx_group_kernel<FP8>"
    timing = "graph"
    traffic_profile = "fp8_linear_config4q_pmc.txt"

    def __init__(self, dev):
        import torch

        from axk import configs

        c = configs.config4_fp8_proj()
        self.host = c
        self.m, self.n, self.k = c["x"].shape[0], c["w"].shape[0], c["w"].shape[1]
        self.alg_bytes = self.n * self.k + 4 * self.n + 2 * self.m * self.k + 2 * self.m * self.n
        self.alg_flops = 2 * self.m * self.n * self.k
        self.copies = max(2, -(-ROTATE_BYTES // (self.n * self.k)))
        w = c["w"].to(dev)
        self.w = [w.clone() for _ in range(self.copies)]
        self.sb = c["scale_b"].to(dev)
        self.x = c["x"].to(dev)
        self.out = torch.empty(self.m, self.n, dtype=torch.bfloat16, device=dev)
        self.config = {"workload": "config4 q projection: FP8 E4M3 linear N=16384 K=4096 M=8 (per-channel scale)",
                       "rotating_copies": self.copies}
        self.dtype = "fp8 e4m3 x bf16 -> fp32 acc"

    def step(self, i: int) -> None:
        import axk

        axk.fp8_gemm(self.x, self.w[i % self.copies], None, self.sb, output=self.out)

    def cpu_baseline(self) -> dict:
        import torch

        from oracle import mx as omx

        c = self.host
        nt = _cpu_threads()
        torch.set_num_threads(nt)
        w = c["w"].numpy()
        sec, reps = _time_cpu(lambda: omx.fp8_linear(c["x"], w, None, c["scale_b"]), budget_s=10.0, min_reps=2)
        return {"value": sec * 1e6, "unit": "µs/op", "cores": nt, "kind": "port",
                "sample": f"full config4 q projection (oracle/mx.py fp8_linear, torch CPU), median of {reps} runs"}


class Int8LinearWorkload(Workload):
    """sgl int8_gemm (gemm.py:479-492) at config 4's q-projection shape: int8 weight [16384, 4096] with an fp32 scale
    per channel, int8 activations [8, 4096] with a scale per row, bf16 out. Algorithmic bytes: weight + both scale
    vectors + activations + out."""

    name = "int8_linear"
    tokens = 8  # tokens one step carries through the path
    kernel = "int8_skinny_kernel<1>"
    timing = "graph"
    traffic_profile = "int8_linear_n16384_pmc.txt"

    def __init__(self, dev):
        import torch

        self.m, self.n, self.k = 8, 16384, 4096
        g = torch.Generator().manual_seed(8)
        self.alg_bytes = self.n * self.k + 4 * self.n + self.m * self.k + 4 * self.m + 2 * self.m * self.n
        self.alg_flops = 2 * self.m * self.n * self.k
        self.copies = max(2, -(-ROTATE_BYTES // (self.n * self.k)))
        self.host_w = torch.randint(-128, 128, (self.n, self.k), generator=g, dtype=torch.int8)
        self.host_x = torch.randint(-128, 128, (self.m, self.k), generator=g, dtype=torch.int8)
        self.host_sa = torch.rand(self.m, generator=g) / 127
        self.host_sb = torch.rand(self.n, generator=g) / (127 * 64)
        w = self.host_w.to(dev)
        self.w = [w.clone() for _ in range(self.copies)]
        self.x, self.sa, self.sb = self.host_x.to(dev), self.host_sa.to(dev), self.host_sb.to(dev)
        self.out = torch.empty(self.m, self.n, dtype=torch.bfloat16, device=dev)
        self.config = {"workload": "int8_gemm N=16384 K=4096 M=8 (per-row and per-channel scales, bf16 out)",
                       "rotating_copies": self.copies}
        self.dtype = "int8 x int8 -> int32 acc"

    def step(self, i: int) -> None:
        import axk

        axk.int8_gemm(self.x, self.w[i % self.copies], self.sa, self.sb, output=self.out)

    def cpu_baseline(self) -> dict:
        import torch

        from oracle import mx as omx

        nt = _cpu_threads()
        torch.set_num_threads(nt)
        w, x, sa, sb = self.host_w.numpy(), self.host_x.numpy(), self.host_sa.numpy(), self.host_sb.numpy()
        sec, reps = _time_cpu(lambda: omx.int8_linear(x, w, sa, sb), budget_s=10.0, min_reps=2)
        return {"value": sec * 1e6, "unit": "µs/op", "cores": nt, "kind": "port",
                "sample": f"the full op (oracle/mx.py int8_linear, torch CPU), median of {reps} runs"}


class Int4LinearWorkload(Workload):
    """sgl int4_gemm (gemm.py:662-677) at config 4's q-projection shape: int4 weight [16384, 4096] one value per byte
    with an fp32 scale per 128 along K, bf16 activations [8, 4096], bf16 out. Algorithmic bytes: weight + group scales
    + activations + out."""

    name = "int4_linear"
    tokens = 8  # tokens one step carries through the path
    kernel = "int4_skinny_kernel<1, 64>"
    timing = "graph"
    traffic_profile = "int4_linear_n16384_pmc.txt"

    def __init__(self, dev):
        import torch

        self.m, self.n, self.k, self.group = 8, 16384, 4096, 128
        g = torch.Generator().manual_seed(4)
        ng = self.k // self.group
        self.alg_bytes = self.n * self.k + 4 * self.n * ng + 2 * self.m * self.k + 2 * self.m * self.n
        self.alg_flops = 2 * self.m * self.n * self.k
        per_copy = self.n * self.k + 4 * self.n * ng
        self.copies = max(2, -(-ROTATE_BYTES // per_copy))
        self.host_w = torch.randint(-8, 8, (self.n, self.k), generator=g, dtype=torch.int8)
        self.host_s = torch.rand(self.n, ng, generator=g) / 512
        self.host_x = torch.randn(self.m, self.k, generator=g).to(torch.bfloat16)
        w, s = self.host_w.to(dev), self.host_s.to(dev)
        self.w = [w.clone() for _ in range(self.copies)]
        self.s = [s.clone() for _ in range(self.copies)]
        self.x = self.host_x.to(dev)
        self.out = torch.empty(self.m, self.n, dtype=torch.bfloat16, device=dev)
        self.config = {"workload": "int4_gemm N=16384 K=4096 M=8 (one int4 per byte, fp32 scale per 128, bf16 out)",
                       "rotating_copies": self.copies}
        self.dtype = "int4 x bf16 -> fp32 acc"

    def step(self, i: int) -> None:
        import axk

        j = i % self.copies
        axk.int4_gemm(self.x, self.w[j], self.s[j], output=self.out)

    def cpu_baseline(self) -> dict:
        import torch

        from oracle import mx as omx

        nt = _cpu_threads()
        torch.set_num_threads(nt)
        w, s = self.host_w.numpy(), self.host_s.numpy()
        sec, reps = _time_cpu(lambda: omx.int4_linear(self.host_x, w, s), budget_s=10.0, min_reps=2)
        return {"value": sec * 1e6, "unit": "µs/op", "cores": nt, "kind": "port",
                "sample": f"the full op (oracle/mx.py int4_linear, torch CPU), median of {reps} runs"}


class KvWriteWorkload(Workload):
    """Config 1's KV write: the current token's K and V rows (16 sequences x 2 KV heads x 256) scattered into the
    paged cache in place. Algorithmic bytes: k, v and the locations read, the rows written."""

    name = "kv_write"
    tokens = 16  # tokens one step carries through the path
    kernel = "paged_kv_write_kernel"
    timing = "graph"
    traffic_profile = "kv_write_config1_pmc.txt"

    def __init__(self, dev):
        from axk import configs

        c = configs.config1_kv_write()
        self.host = c
        b, hkv, d = c["k"].shape
        self.alg_bytes = 2 * (2 * b * hkv * d * 2) + c["loc"].numel() * 4
        self.cache = c["cache"].to(dev)
        self.k, self.v, self.loc = c["k"].to(dev), c["v"].to(dev), c["loc"].to(dev)
        self.config = {"workload": "config1 KV write: B=16 HKV=2 D=256 page=64, rows into the paged cache"}
        self.dtype = "bf16 rows"

    def step(self, i: int) -> None:
        from axk import attention

        attention.store_paged_kv(self.k, self.v, self.cache, self.loc)

    def cpu_baseline(self) -> dict:
        from oracle import paged_attn as opa

        c = self.host
        cache = c["cache"].clone()
        loc = c["loc"].numpy()
        sec, reps = _time_cpu(lambda: opa.store_paged_kv_(cache, c["k"], c["v"], loc), budget_s=2.0, min_reps=20,
                              max_reps=2000)
        return {"value": sec * 1e6, "unit": "µs/op", "cores": 1, "kind": "port",
                "sample": f"full config1 KV write into the config1 cache (oracle/paged_attn.py store_paged_kv_, in "
                          f"place), median of {reps} runs"}


class GroupDecodeWorkload(Workload):
    """Config 4: the 16-layer hybrid decode group ((GDN, GDN, GDN, attention) x 4), batch 8, every sequence at
    131,072 tokens of paged bf16 KV; FP8 projections, MXFP4 MLP (inter 12288), hidden 4096. One step = the 16
    layers (each about 15 launches) for one new token per sequence, captured with the other steps in one HIP
    graph. value: µs per decode layer (step / 16). Algorithmic bytes: every weight and norm read once, the GDN
    and conv states read and written, every sequence's K and V read by each attention layer, the new rows written.
    The inputs (about 20 GB) are generated on the device by a seeded device generator."""

    name = "group_decode"
    tokens = 8  # tokens one step carries through the path
    kernel = "hybrid decode group (16 layers)"
    timing = "graph"
    traffic_profile = "group_decode_config4_pmc.txt"

    def __init__(self, dev):
        import torch

        from axk import configs, layer

        c = configs.config4_group(dev)
        c4 = c["cfg"]
        self.c, self.c4 = c, c4
        b, h, f = c4["batch"], c4["hidden"], c4["inter"]
        self.ws_g = layer.gdn_workspace(b, h, c4["nk"], c4["nv"], f, dev)
        self.ws_a = layer.attn_workspace(b, h, c4["hq"], c4["hkv"], c4["d"], f, dev)
        self.buf = [c["x"].clone(), torch.empty_like(c["x"])]
        wbytes = sum(t.numel() * t.element_size() for L in c["layers"] for t in L["w"].values())
        sbytes = sum(2 * (L["state"].numel() * 4 + L["conv"].numel() * 2) for L in c["layers"] if L["kind"] == "g")
        tokens = b * (c4["ctx"] + 1)
        n_attn = sum(1 for L in c["layers"] if L["kind"] == "a")
        kv_row = 2 * c4["hkv"] * c4["d"] * 2  # K and V of one token, bytes
        self.alg_bytes = wbytes + sbytes + n_attn * (tokens * kv_row + b * kv_row) + 2 * len(c["layers"]) * b * h * 2
        self.layers_per_step = len(c["layers"])
        self.value_per = self.layers_per_step
        self.unit = "µs/decode-layer"
        self.config = {"workload": "config4: 16-layer hybrid decode group (ggga x4), B=8, ctx 131072, H=4096, "
                                   "HQ=32 HKV=4 D=256, GDN 16/32 heads, FP8 projections, MXFP4 MLP F=12288",
                       "layers": self.layers_per_step, "kv_bytes_per_attention_layer": tokens * kv_row}
        self.dtype = "bf16 activations, fp8 / mxfp4 weights, fp32 accumulation and state"

    def step(self, i: int) -> None:
        from axk import layer

        c, c4 = self.c, self.c4
        x, y = self.buf
        for L in c["layers"]:
            if L["kind"] == "g":
                layer.gdn_layer_decode(x, L["w"], L["state"], L["conv"], c4["nk"], c4["nv"], c4["eps"],
                                       workspace=self.ws_g, out=y, state_out=L["state"], conv_out=L["conv"])
            else:
                layer.attn_layer_decode(x, L["w"], c["cos"], c["sin"], L["cache"], c["indptr"], c["indices"],
                                        c["last_page_len"], c["loc"], c4["hq"], c4["rot"], c4["eps"],
                                        workspace=self.ws_a, out=y)
            x, y = y, x

    def cpu_baseline(self) -> dict:
        import torch

        from oracle import layer as olayer

        c, c4 = self.c, self.c4
        nt = _cpu_threads()
        torch.set_num_threads(nt)
        gl = next(L for L in c["layers"] if L["kind"] == "g")
        al = next(L for L in c["layers"] if L["kind"] == "a")
        wg = {k: v.cpu() for k, v in gl["w"].items()}
        wa = {k: v.cpu() for k, v in al["w"].items()}
        x = c["x"].cpu()
        st, cv = gl["state"].cpu(), gl["conv"].cpu()
        t_g, reps_g = _time_cpu(lambda: olayer.gdn_layer_decode(x, wg, st, cv, c4["nk"], c4["nv"], c4["eps"]),
                                budget_s=8.0, min_reps=1, max_reps=3)
        # sequence 0 of one attention layer at the full context: its pages gathered into a compact host cache
        n0 = int(c["indptr"][1].item())
        pages = c["indices"][:n0].long()
        cache0 = al["cache"][pages].cpu()
        ind0 = torch.arange(n0, dtype=torch.int32)
        ptr0 = torch.tensor([0, n0], dtype=torch.int32)
        loc0 = torch.tensor([[n0 - 1, int(c["loc"][0, 1].item())]], dtype=torch.int32)
        t_a, reps_a = _time_cpu(lambda: olayer.attn_layer_decode(x[:1], wa, c["cos"][:1].cpu(), c["sin"][:1].cpu(),
                                                                 cache0, ptr0, ind0, c["last_page_len"][:1].cpu(),
                                                                 loc0, c4["hq"], c4["rot"], c4["eps"]),
                                budget_s=8.0, min_reps=1, max_reps=3)
        n_g = sum(1 for L in c["layers"] if L["kind"] == "g")
        n_a = len(c["layers"]) - n_g
        step = n_g * t_g + n_a * c4["batch"] * t_a
        return {"value": step / len(c["layers"]) * 1e6, "unit": "µs/decode-layer", "cores": nt, "kind": "port",
                "sample": f"one GDN layer at batch {c4['batch']} (median of {reps_g}) and one attention layer for one "
                          f"sequence at the full context (median of {reps_a}) with the oracle (oracle/layer.py, torch "
                          f"CPU), scaled to {n_g} GDN + {n_a} attention layers x {c4['batch']} sequences, per layer"}


class MoeGroupDecodeWorkload(Workload):
    """The 35B's MoE decode group (qwen35moe_group8_gggaggga_mx8_kvc_c16384, q35_moe_group.py:90-123): 8 layers
    ((GDN, GDN, GDN, attention) x 2) at the 35B's widths, every MLP the MoE block (shared expert MXFP8 inter 512,
    256 MXFP4 experts of 512, top-8), MXFP8 projections, GDN 16 / 32 heads, attention HQ 16 / HKV 2 / D 256; 32
    sequences, each at 16,383 cached tokens of paged bf16 KV (the step's token fills the reference's 16,384-token
    cache). One step = the 8 layers for one new token per sequence (axk.DecodeGroup.step), captured with the other
    steps in one HIP graph. value: µs per decode layer (step / 8). Algorithmic bytes: every dense weight, norm,
    router and shared-expert gate read once, the routed experts each layer actually uses (its distinct experts over
    the 32 tokens), the GDN and conv states read and written, every sequence's K and V read by each attention layer,
    the new rows written, each layer's activations in and out. The inputs (about 6 GB) are generated on the device."""

    name = "moe_group_decode"
    tokens = 32  # tokens one step carries through the path
    kernel = "35B MoE decode group (8 layers)"
    timing = "graph"
    traffic_profile = "moe_group_decode_b32_pmc.txt"  # every kernel of the step, summed

    def __init__(self, dev):
        import torch

        from axk import configs, group

        c = configs.moe_group(dev)
        cg = c["cfg"]
        self.c, self.cg = c, cg
        b, h = cg["batch"], cg["hidden"]
        args = (c["layers"], b, h, dev, cg["nk"], cg["nv"], cg["hq"], cg["rot"], cg["eps"], "mxfp8", "mxfp8")
        # one eager step with the routing outputs kept: the distinct experts each layer reads
        probe = group.DecodeGroup(*args, attn=c["attn"], routing=True)
        probe.step(c["x"])
        self.active = [int(torch.unique(r["topk_ids"]).numel()) for r in probe.routing]
        del probe
        self.grp = group.DecodeGroup(*args, attn=c["attn"])
        self.grp.x.copy_(c["x"])
        per_expert = sum(c["layers"][0]["moe"][n][0].numel() for n in ("e_gw", "e_gs", "e_dw", "e_ds"))
        wbytes = sum(t.numel() * t.element_size() for L in c["layers"] for t in L["w"].values())
        wbytes += sum(L["moe"][n].numel() * L["moe"][n].element_size() for L in c["layers"]
                      for n in ("w_router", "w_shg"))
        sbytes = sum(2 * (L["state"].numel() * 4 + L["conv"].numel() * 2) for L in c["layers"] if L["kind"] == "g")
        tokens = b * (cg["ctx"] + 1)
        n_attn = sum(1 for L in c["layers"] if L["kind"] == "a")
        kv_row = 2 * cg["hkv"] * cg["d"] * 2  # K and V of one token, bytes
        self.alg_bytes = wbytes + sum(self.active) * per_expert + sbytes + \
            n_attn * (tokens * kv_row + b * kv_row) + 2 * len(c["layers"]) * b * h * 2
        self.layers_per_step = len(c["layers"])
        self.value_per = self.layers_per_step
        self.unit = "µs/decode-layer"
        self.config = {"workload": "35B MoE decode group (gggaggga), B=32, ctx 16384, H=2048, MXFP8 projections, "
                                   "GDN 16/32 heads, HQ=16 HKV=2 D=256, MoE 256 MXFP4 experts F=512 top-8 + shared "
                                   "MXFP8 F=512",
                       "layers": self.layers_per_step, "distinct_experts_per_layer": self.active,
                       "kv_bytes_per_attention_layer": tokens * kv_row}
        self.dtype = "bf16 activations, mxfp8 / mxfp4 weights, fp32 accumulation and state"

    def step(self, i: int) -> None:
        self.grp.step()

    def cpu_baseline(self) -> dict:
        import torch

        from oracle import layer as olayer

        c, cg = self.c, self.cg
        nt = _cpu_threads()
        torch.set_num_threads(nt)
        n = 4  # a bounded sample: 4 of the 32 sequences through one GDN layer, scaled by sequences
        gl = next(L for L in c["layers"] if L["kind"] == "g")
        al = next(L for L in c["layers"] if L["kind"] == "a")
        wg = {k: v.cpu() for k, v in gl["w"].items()}
        wa = {k: v.cpu() for k, v in al["w"].items()}
        mg = {k: (v.cpu() if torch.is_tensor(v) else v) for k, v in gl["moe"].items()}
        ma = {k: (v.cpu() if torch.is_tensor(v) else v) for k, v in al["moe"].items()}
        x = c["x"].cpu()
        st, cv = gl["state"][:n].cpu(), gl["conv"][:n].cpu()

        def run_g():
            y, _, _ = olayer.gdn_layer_half(x[:n], wg, st, cv, cg["nk"], cg["nv"], cg["eps"], proj_fmt="mxfp8")
            return olayer.moe_block_parts(x[:n], y, wg, mg, cg["eps"], fmt="mxfp8")

        t_g, reps_g = _time_cpu(run_g, budget_s=8.0, min_reps=1, max_reps=3)
        # sequence 0 of one attention layer at the full context: its pages gathered into a compact host cache
        a = c["attn"]
        n0 = int(a["indptr"][1].item())
        cache0 = al["cache"][a["indices"][:n0].long()].cpu()
        ptr0 = torch.tensor([0, n0], dtype=torch.int32)
        ind0 = torch.arange(n0, dtype=torch.int32)
        loc0 = torch.tensor([[n0 - 1, int(a["loc"][0, 1].item())]], dtype=torch.int32)
        cos, sin, last = a["cos"][:1].cpu(), a["sin"][:1].cpu(), a["last_page_len"][:1].cpu()

        def run_a():
            y, _ = olayer.attn_layer_half(x[:1], wa, cos, sin, cache0, ptr0, ind0, last, loc0, cg["hq"], cg["rot"],
                                          cg["eps"], proj_fmt="mxfp8")
            return olayer.moe_block_parts(x[:1], y, wa, ma, cg["eps"], fmt="mxfp8")

        t_a, reps_a = _time_cpu(run_a, budget_s=8.0, min_reps=1, max_reps=3)
        n_g = sum(1 for L in c["layers"] if L["kind"] == "g")
        n_a = len(c["layers"]) - n_g
        step = n_g * t_g * cg["batch"] / n + n_a * cg["batch"] * t_a
        return {"value": step / len(c["layers"]) * 1e6, "unit": "µs/decode-layer", "cores": nt, "kind": "port",
                "sample": f"one GDN MoE layer on {n} of the {cg['batch']} sequences (median of {reps_g}) and one "
                          f"attention MoE layer for one sequence at the full context (median of {reps_a}) with the "
                          f"oracle (oracle/layer.py, torch CPU), scaled to {n_g} GDN + {n_a} attention layers x "
                          f"{cg['batch']} sequences, per layer"}


WORKLOADS = {MxLinearWorkload.name: MxLinearWorkload, PagedDecodeWorkload.name: PagedDecodeWorkload,
             GdnDecodeWorkload.name: GdnDecodeWorkload, GdnPrefillWorkload.name: GdnPrefillWorkload,
             MoeDecodeWorkload.name: MoeDecodeWorkload, MoePrefillWorkload.name: MoePrefillWorkload,
             MxDequantWorkload.name: MxDequantWorkload, Fp8LinearWorkload.name: Fp8LinearWorkload,
             KvWriteWorkload.name: KvWriteWorkload, GroupDecodeWorkload.name: GroupDecodeWorkload,
             LmHeadWorkload.name: LmHeadWorkload, LmHeadNvfp4Workload.name: LmHeadNvfp4Workload, PagedDecodeFp8Workload.name: PagedDecodeFp8Workload, PagedDecodeI8Workload.name: PagedDecodeI8Workload,
             PagedPrefillWorkload.name: PagedPrefillWorkload, MoeLayerDecodeWorkload.name: MoeLayerDecodeWorkload,
             MxLinearPrefillWorkload.name: MxLinearPrefillWorkload, MoeLayerPrefillWorkload.name: MoeLayerPrefillWorkload,
             MoeGroupDecodeWorkload.name: MoeGroupDecodeWorkload, Int8LinearWorkload.name: Int8LinearWorkload,
             Int4LinearWorkload.name: Int4LinearWorkload, CopyCalibWorkload.name: CopyCalibWorkload}
DEFAULT_WORKLOAD = PagedDecodeWorkload.name


WARM_GPU_MS = 200.0  # untimed graph replays before the timed one: the clocks settle after the first launches


def _graph_ms(fn, steps: int) -> float:
    """ms per call of fn over exactly `steps` calls captured as one HIP graph; the graph is replayed untimed (upload,
    clocks) for about WARM_GPU_MS first, then one replay is timed with HIP events on the graph's own stream."""
    import torch

    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for i in range(steps):
                fn(i)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    spent = 0.0
    for _ in range(50):
        t0 = time.perf_counter()
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        spent += (time.perf_counter() - t0) * 1e3
        if spent >= WARM_GPU_MS:
            break
    start.record(stream)
    with torch.cuda.stream(stream):
        graph.replay()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def measure(wl, steps: int, warmup: int, eager: bool = False) -> tuple[float, float]:
    """(ms per step, ms per launch of the workload's roofline kernel) over exactly `steps` timed steps.
    eager: launch every step on the stream even where the workload is normally timed as one HIP graph."""
    import torch

    torch.cuda.synchronize()
    for i in range(warmup):
        wl.step(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if wl.timing == "graph" and not eager:
        # exactly K steps in one HIP graph (no host launch overhead in the measurement)
        ms_per_step = _graph_ms(wl.step, steps)
        roof = getattr(wl, "roofline_step", None)
        if roof is None:
            return ms_per_step, ms_per_step
        # the roofline kernel on its own: K launches of it (over the same rotating inputs) as one HIP graph
        return ms_per_step, _graph_ms(roof, steps)
    # Eager steps on the current stream; HIP events bracket every launch of the dominant kernel.
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    start.record()
    for i in range(steps):
        wl.pre(i)
        evs[i][0].record()
        wl.main(i)
        evs[i][1].record()
        wl.post(i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps, sum(a.elapsed_time(b) for a, b in evs) / steps


def report_line(wl, args, ms_per_step: float, kernel_ms: float) -> dict:
    achieved = wl.alg_bytes / (kernel_ms * 1e-3) / 1e9
    if getattr(wl, "mfma", False):  # MFMA-bound: the roofline is the dense bf16 rate
        tf = wl.alg_flops / (kernel_ms * 1e-3) / 1e12
        roof = {"bound": "mfma", "kernel": wl.kernel, "achieved": round(tf, 2), "peak": BF16_PEAK_TFS,
                "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFS, 4), "traffic": read_traffic(wl),
                "alg_flops_per_launch": wl.alg_flops, "alg_bytes_per_launch": wl.alg_bytes, **mfma_fracs(tf)}
    else:
        roof = {"bound": "hbm", "kernel": wl.kernel, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic(wl),
                "alg_bytes_per_launch": wl.alg_bytes}
    per = getattr(wl, "value_per", 1)  # steps report per op, the decode group per layer
    return {
        "metric": METRIC,
        "value": round(ms_per_step * 1e3 / per, 3),
        "unit": getattr(wl, "unit", "µs/op"),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl.dtype,
        "data": "synthetic (seeded generators in axk/configs.py)",
        "config": wl.config,
        "kernel_us": round(kernel_ms * 1e3, 3),
        "achieved_gbs": round(achieved, 1),
        "hbm_frac": round(achieved / HBM_PEAK_GBS, 4),
        "tokens_per_s": tokens_per_s(wl, ms_per_step),
        "roofline": roof,
    }


def read_traffic(wl):
    """HBM bytes per launch of the roofline kernel, from the committed PMC summary (FETCH_SIZE + WRITE_SIZE
    per dispatch, scaled by the copy-kernel calibration factor), or None when no summary exists."""
    if not wl.traffic_profile:
        return None
    path = os.path.join(ROOT, "profiles", wl.traffic_profile)
    try:
        with open(path, encoding="utf-8") as f:
            for ln in f:
                if ln.startswith("traffic_bytes_per_launch:"):
                    return int(float(ln.split(":", 1)[1]))
    except OSError:
        return None
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default=DEFAULT_WORKLOAD, choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-suite", action="store_true", help="measure only the headline workload")
    ap.add_argument("--eager", action="store_true", help="no HIP graph capture (for counter collection)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        return 2

    import torch

    import axk

    axk.load_library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    wl = WORKLOADS[args.workload](dev)
    ms_per_step, kernel_ms = measure(wl, args.steps, args.warmup, args.eager)
    line = report_line(wl, args, ms_per_step, kernel_ms)
    if not args.no_suite:
        # the other hot-path workloads, measured in the same process (reported beside the headline line)
        suite = {}
        for name, cls in WORKLOADS.items():
            if name == args.workload or not cls.in_suite:
                continue
            other = cls(dev)
            ms, kms = measure(other, max(20, args.steps // 4), min(args.warmup, 10), args.eager)
            gbs = other.alg_bytes / (kms * 1e-3) / 1e9
            suite[name] = {"us_per_op": round(ms * 1e3, 3), "kernel_us": round(kms * 1e3, 3),
                           "achieved_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                           "tokens_per_s": tokens_per_s(other, ms), "config": other.config["workload"]}
            if getattr(other, "value_per", 1) > 1:
                suite[name]["us_per_decode_layer"] = round(ms * 1e3 / other.value_per, 3)
            if getattr(other, "mfma", False):
                tf = other.alg_flops / (kms * 1e-3) / 1e12
                suite[name].update({"achieved_tflops": round(tf, 2), **mfma_fracs(tf)})
            del other
            torch.cuda.empty_cache()
        line["suite"] = suite
    if not args.no_cpu:
        cpu = wl.cpu_baseline()
        if cpu is not None:
            cpu.update(cpu_machine())
            if wl.tokens and cpu.get("value"):  # the same step on the host: value is per op (per layer for a group)
                cpu["tokens_per_s"] = round(wl.tokens / (cpu["value"] * 1e-6 * getattr(wl, "value_per", 1)), 3)
            line["cpu_baseline"] = cpu
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
