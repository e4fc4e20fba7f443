"""axk — MI355X (gfx950) kernels for the per-layer Qwen3.5 decode/prefill hot path of ax-dsl-kernels.

Python host layer over libaxk.so (include/axk.h). Operator names and contracts mirror the reference's
sgl_kernel_axera operator API; tensors are torch device tensors used only as memory and streams.
"""
from . import _lib
from .gemm import bf16_gemm, fp8_gemm, int4_gemm, int8_gemm, mxfp4_dequant, mxfp4_gemm, mxfp8_gemm, nvfp4_gemm
from .quantization import quantize_nvfp4

__all__ = ["bf16_gemm", "fp8_gemm", "int4_gemm", "int8_gemm", "mxfp4_dequant", "mxfp4_gemm", "mxfp8_gemm",
           "nvfp4_gemm", "quantize_nvfp4", "load_library"]


def load_library():
    """Load libaxk.so (raises ImportError if it has not been built)."""
    return _lib.load()

from . import attention  # noqa: E402
from .attention import (  # noqa: E402
    paged_attention_decode,
    paged_decode,
    paged_decode_plan,
    paged_decode_run,
    paged_decode_workspace,
    store_paged_kv,
    paged_decode_fp8,
    store_paged_kv_fp8,
    paged_decode_i8,
    store_paged_kv_i8,
    paged_prefill,
)

__all__ += ["attention", "paged_attention_decode", "paged_decode", "paged_decode_plan", "paged_decode_run", "paged_decode_workspace",
            "store_paged_kv", "paged_decode_fp8", "store_paged_kv_fp8", "paged_decode_i8", "store_paged_kv_i8",
            "paged_prefill"]

from . import gdn  # noqa: E402
from .gdn import gdn_chunk_prefill, gdn_chunk_workspace, gdn_recurrent  # noqa: E402

__all__ += ["gdn", "gdn_chunk_prefill", "gdn_chunk_workspace", "gdn_recurrent"]

from . import moe  # noqa: E402
from .moe import moe_decode, moe_experts, moe_route, moe_workspace  # noqa: E402

__all__ += ["moe", "moe_decode", "moe_experts", "moe_route", "moe_workspace"]

from . import glue  # noqa: E402

__all__ += ["glue"]

from . import layer  # noqa: E402

__all__ += ["layer"]

from . import group  # noqa: E402
from .group import DecodeGroup  # noqa: E402

__all__ += ["group", "DecodeGroup"]

from . import manifest  # noqa: E402
from .manifest import Manifest, io_table  # noqa: E402

__all__ += ["manifest", "Manifest", "io_table"]
