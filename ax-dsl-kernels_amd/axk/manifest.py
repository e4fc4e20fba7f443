"""The reference's deliverable format, bound to the axk entry points: manifest.json, .layout packs and IO tables.

manifest.json (tools/manifest/mkmanifest.py:296-311) lists per role a kernel's file and its IO as
{name, bytes, dtype, shape}, and for packed kernels the packs and their members (mkmanifest.py:254-277, the .layout
lines "member pack offset bytes [column split]"). A layer's parameters live in one pack per dtype (pw E4M3, ps E8M0,
pf f32, pb bf16, p4 E2M1 pairs: models/qwen38_27b/decode/q35_layer_pk.py:1-12, 32-45), each member at a 64-byte
aligned byte offset. The weights the board's cores split by columns (w_out / w_o / w_down and their scales) are stored
column block after column block: "blk rows cols width" equal strips (q35_layer_pk.py:108-125) or explicit byte ranges
(models/qwen35_35b_a3b/src/70b0fbc/q35_layer_mc.py:1236-1296, 1323-1336). The 9B whole-model group reads its row-split
projections from per-phase banks k_b<phase>_<name>[block], layer j = 4 block + phase
(models/qwen35_9b/whole/src/q35_group.py:60-76, 293-303).

Binding a layer returns its parameters under the names the axk layer entry points take (axk.layer): plain members as
views of the caller's pack buffers (no copy); column-split members and the GDN's q / k / v bank parts assembled once
into row-major weights, because the axk kernels stream row-major [N, K] rows. io_table() answers the IO of the roles
libaxk serves from the library itself (axk_io_table).
"""
from __future__ import annotations

import ctypes
import json
import re
from dataclasses import dataclass, field
from typing import Optional

import torch

from . import _lib

ALIGN = 64  # member offsets in a pack (q35_layer_pk.py ALIGN)
PACKS = ("p4", "pw", "ps", "pf", "pb")
# AX dtype code -> the torch dtype axk takes the storage as (E4M3 / E5M2 / E2M1 / E8M0 as bytes)
DT_TORCH = {1: torch.uint8, 3: torch.float32, 6: torch.int32, 9: torch.bfloat16, 10: torch.float16, 11: torch.uint8,
            12: torch.uint8, 15: torch.uint8}
DT_SIZE = {1: 1, 3: 4, 6: 4, 9: 2, 10: 2, 11: 1, 12: 1}  # bytes per element; 15 (E2M1) is half a byte

# bank input k_b<phase>_<name> -> the parameter it holds, per layer kind (q35_group.py:66-73); the GDN's w_qkv is
# banked as its q / k / v row blocks (gq / gk / gv), joined again on binding
BANKS = {
    "gdn": {"attn_w_q": "w_gq", "attn_w_q_scale": "s_gq", "attn_w_k": "w_gk", "attn_w_k_scale": "s_gk",
            "attn_w_v": "w_gv", "attn_w_v_scale": "s_gv", "attn_w_z": "w_z", "attn_w_z_scale": "s_z",
            "attn_w_a": "w_a", "attn_w_b": "w_b", "mlp_w1": "w_gate", "mlp_w_scale1": "s_gate", "mlp_w2": "w_up",
            "mlp_w_scale2": "s_up"},
    "attn": {"attn_w_q": "w_q", "attn_w_scale_q": "s_q", "attn_w_k": "w_k", "attn_w_scale_k": "s_k",
             "attn_w_v": "w_v", "attn_w_scale_v": "s_v", "mlp_w1": "w_gate", "mlp_w_scale1": "s_gate",
             "mlp_w2": "w_up", "mlp_w_scale2": "s_up"},
}
EXPERT_IO = ("e_gw", "e_gs", "e_dw", "e_ds")


def check_dtype(dtype: int, name: Optional[str] = None) -> None:
    """Raise ValueError naming the IO for an AX dtype code axk does not take (0: the committed 35B manifest gives it to
    its bf16 KV-cache outputs; the reference's ONNX table, tools/manifest/onnx_io.py:18-29, has no entry for it)."""
    if dtype not in DT_TORCH:
        raise ValueError(f"IO {name or '?'}: AX dtype code {dtype} is not one axk handles ({sorted(DT_TORCH)})")


def storage_bytes(dtype: int, shape, name: Optional[str] = None) -> int:
    check_dtype(dtype, name)
    n = 1
    for d in shape:
        n *= int(d)
    return n // 2 if dtype == 15 else n * DT_SIZE[dtype]


def storage_shape(dtype: int, shape) -> tuple:
    """The shape of the stored elements (E2M1: pairs along the last dimension)."""
    shape = tuple(int(d) for d in shape)
    return shape[:-1] + (shape[-1] // 2,) if dtype == 15 else shape


@dataclass(frozen=True)
class IoEntry:
    """One IO of a kernel: the AX engine's IO meta (tools/board/iojson.c:23-34)."""
    name: str
    bytes: int
    dtype: int
    shape: tuple

    @classmethod
    def of(cls, e) -> "IoEntry":
        if isinstance(e, dict):
            return cls(e["name"], int(e["bytes"]), int(e["dtype"]), tuple(int(d) for d in e["shape"]))
        n, b, t, s = e
        return cls(n, int(b), int(t), tuple(int(d) for d in s))

    def as_list(self) -> list:
        return [self.name, self.bytes, self.dtype, list(self.shape)]


@dataclass(frozen=True)
class Member:
    """A member of a pack: `bytes` bytes at byte `offset` of pack `pack`. strips (rows, row bytes, strip bytes) or
    blocks (rows, row bytes, ((a, b), ...) byte ranges of a row) describe a column-split weight stored block after
    block, each block [rows, b - a] row-major."""
    name: str
    pack: str
    offset: int
    bytes: int
    param: str
    layer: Optional[int] = None
    kind: Optional[str] = None
    strips: Optional[tuple] = None
    blocks: Optional[tuple] = None

    @classmethod
    def of(cls, d: dict) -> "Member":
        bl = d.get("blocks")
        return cls(d["name"], d["pack"], int(d["offset"]), int(d["bytes"]), d.get("param", d["name"]), d.get("layer"),
                   d.get("kind"), tuple(d["strips"]) if d.get("strips") else None,
                   (int(bl["rows"]), int(bl["row_bytes"]), tuple((int(a), int(b)) for a, b in bl["ranges"]))
                   if bl else None)

    def column_ranges(self) -> Optional[tuple]:
        """(rows, row bytes, byte ranges in storage order) of a column-split member, else None."""
        if self.strips:
            rows, cols, width = self.strips
            return rows, cols, tuple((a, a + width) for a in range(0, cols, width))
        return self.blocks

    def to_row_major(self, raw: torch.Tensor) -> torch.Tensor:
        """raw: this member's bytes (u8 [bytes]) -> u8 [rows, row bytes] row-major (a new tensor for a column-split
        member, raw itself otherwise)."""
        cr = self.column_ranges()
        if cr is None:
            return raw
        rows, row_bytes, ranges = cr
        out = torch.empty(rows, row_bytes, dtype=torch.uint8, device=raw.device)
        o = 0
        for a, b in ranges:
            n = rows * (b - a)
            out[:, a:b] = raw[o:o + n].view(rows, b - a)
            o += n
        return out

    def from_row_major(self, w: torch.Tensor) -> torch.Tensor:
        """The stored bytes (u8 [bytes]) of a row-major u8 [rows, row bytes] weight: the inverse of to_row_major."""
        cr = self.column_ranges()
        if cr is None:
            return w.reshape(-1)
        _, _, ranges = cr
        return torch.cat([w[:, a:b].reshape(-1) for a, b in ranges])


def parse_layout(text: str) -> tuple[dict, list]:
    """A .layout file (q35_layer_mc.py:1323-1336, q35_layer_pk.py:275-279): "pack - 0 bytes" lines size the packs;
    "member pack offset bytes" lines place members, optionally followed by "blk rows cols width" (equal column strips)
    or "rows row_bytes a:b,c:d,..." (column blocks); members L<j>.<param> belong to layer j (mkmanifest.py:254-277).
    Returns (packs {name: bytes}, [Member])."""
    packs, members = {}, []
    for line in text.splitlines():
        f = line.split()
        if len(f) < 4:
            continue
        name, pack, off, nbytes = f[0], f[1], int(f[2]), int(f[3])
        if pack == "-":
            packs[name] = nbytes
            continue
        lm = re.match(r"L(\d+)\.(.+)", name)
        layer, param = (int(lm.group(1)), lm.group(2)) if lm else (None, name)
        rest = f[4:]
        strips = blocks = None
        if rest[:1] == ["blk"]:
            strips = tuple(int(x) for x in rest[1:4])
        elif len(rest) >= 3:
            blocks = (int(rest[0]), int(rest[1]),
                      tuple((int(a), int(b)) for a, b in (r.split(":") for r in rest[2].split(","))))
        members.append(Member(name, pack, off, nbytes, param, layer, None, strips, blocks))
    return packs, members


@dataclass
class Kernel:
    """One role of a manifest: the kernel file, its IO and (packed kernels) packs and members."""
    role: str
    file: str
    inputs: list
    outputs: list
    packs: dict = field(default_factory=dict)
    members: list = field(default_factory=list)

    def entry(self, name: str) -> IoEntry:
        for e in self.inputs + self.outputs:
            if e.name == name:
                return e
        raise KeyError(f"{self.role}: no IO named {name}")

    def io_table(self) -> dict:
        """{"in": [[name, bytes, dtype, shape], ...], "out": [...]} as iojson prints it."""
        return {"in": [e.as_list() for e in self.inputs], "out": [e.as_list() for e in self.outputs]}

    def check_buffers(self, buffers: dict, names=None) -> None:
        """Every IO of the kernel (or only `names`) present in buffers with the kernel's byte count, and contiguous:
        the name -> bytes check of models/qwen35_35b_a3b/sgl/scripts/check_adapter_abi.py:20-56. Raises ValueError
        listing every mismatch."""
        bad = []
        for e in self.inputs + self.outputs:
            if names is not None and e.name not in names:
                continue
            t = buffers.get(e.name)
            if t is None:
                bad.append(f"{e.name}: missing")
                continue
            nb = t.numel() * t.element_size()
            if nb != e.bytes:
                bad.append(f"{e.name}: {nb} bytes, the kernel's IO has {e.bytes}")
            elif not t.is_contiguous():
                bad.append(f"{e.name}: not contiguous")
        if bad:
            raise ValueError(f"{self.role} ({self.file}): " + "; ".join(bad))

    def layer_members(self, layer: int) -> list:
        return [m for m in self.members if m.layer == layer]

    def kinds(self) -> list:
        """The layer kinds of a group kernel in layer order ("gdn" / "attn"): from the members' kind, else from the
        file name's pattern (..._group<G>_<g|a ...>_...)."""
        kinds = {}
        for m in self.members:
            if m.layer is not None and m.kind:
                kinds[m.layer] = m.kind
        pat = re.search(r"_group\d+_([ga]+)_", self.file)
        if pat:
            for j, c in enumerate(pat.group(1)):
                kinds.setdefault(j, "gdn" if c == "g" else "attn")
        return [kinds[j] for j in sorted(kinds)]


def _u8(t: torch.Tensor) -> torch.Tensor:
    if not t.is_contiguous():
        raise ValueError("a pack or bank buffer must be contiguous")
    return t.reshape(-1).view(torch.uint8)


def _typed(raw: torch.Tensor, dtype: int, shape, name: Optional[str] = None) -> torch.Tensor:
    """u8 storage -> the tensor axk takes for an IO of AX dtype `dtype` and logical shape `shape`."""
    check_dtype(dtype, name)
    return raw.view(DT_TORCH[dtype]).view(storage_shape(dtype, shape))


def weight_format(params: dict, name: str) -> str:
    """The axk weight format ("fp8" / "mxfp8" / "mxfp4") of the manifest parameter w_<name> with its scales s_<name>:
    E2M1 elements -> "mxfp4"; E4M3 with E8M0 scales -> "mxfp8"; E4M3 with f32 per-channel scales -> "fp8"."""
    w, s = params["w_" + name], params["s_" + name]
    if w.dtype == 15:
        return "mxfp4"
    if w.dtype == 11:
        return "mxfp8" if s.dtype == 1 else "fp8"
    raise ValueError(f"w_{name}: dtype {w.dtype} is not a weight format axk reads")


@dataclass
class LayerParams:
    """A bound layer: its kind, its parameters under axk.layer's names (w_router / w_shg and the routed experts
    e_gw / e_gs / e_dw / e_ds of a MoE layer with them), and the weight formats of its projections and MLP."""
    kind: str
    weights: dict
    proj_fmt: str
    mlp_fmt: str


class Manifest:
    """A parsed manifest.json (format 1)."""

    def __init__(self, d: dict):
        if d.get("format") != 1:
            raise ValueError(f"manifest format {d.get('format')} is not 1")
        self.model = d.get("model")
        self.context = d.get("context")
        self.cores = d.get("cores")
        self.params = {kind: {n: IoEntry(n, int(p["bytes"]), int(p["dtype"]), tuple(p["shape"]))
                              for n, p in ps.items()} for kind, ps in d.get("params", {}).items()}
        self.kernels = {}
        for role, k in d.get("kernels", {}).items():
            self.kernels[role] = Kernel(role, k["file"], [IoEntry.of(e) for e in k["in"]],
                                        [IoEntry.of(e) for e in k["out"]], dict(k.get("packs", {})),
                                        [Member.of(m) for m in k.get("members", [])])

    @classmethod
    def load(cls, path: str) -> "Manifest":
        with open(path) as f:
            return cls(json.load(f))

    def kernel(self, role: str) -> Kernel:
        if role not in self.kernels:
            raise ValueError(f"manifest of {self.model}: no role {role!r} (roles: {sorted(self.kernels)})")
        return self.kernels[role]

    def check_members(self, role: str) -> None:
        """The packed kernel's members are consistent with its packs and the manifest's parameters: each member inside
        its pack, at a 64-byte aligned offset, not overlapping another member of its pack, of the parameter's storage
        bytes; a column split covers every byte of a row exactly once. Raises ValueError listing every problem."""
        k = self.kernel(role)
        bad = []
        by_pack = {}
        for m in k.members:
            size = k.packs.get(m.pack)
            if size is None:
                bad.append(f"{m.name}: pack {m.pack} not sized")
                continue
            if m.offset % ALIGN or m.offset < 0 or m.offset + m.bytes > size:
                bad.append(f"{m.name}: [{m.offset}, +{m.bytes}) not a 64-byte aligned range of {m.pack} ({size})")
            by_pack.setdefault(m.pack, []).append((m.offset, m.offset + m.bytes, m.name))
            p = self.params.get(m.kind or "", {}).get(m.param)
            if p is not None and p.bytes != m.bytes:
                bad.append(f"{m.name}: {m.bytes} bytes, the parameter has {p.bytes}")
            cr = m.column_ranges()
            if cr is not None:
                rows, row_bytes, ranges = cr
                cover = sorted(ranges)
                if rows * row_bytes != m.bytes or cover[0][0] != 0 or cover[-1][1] != row_bytes or any(
                        a[1] != b[0] for a, b in zip(cover, cover[1:])):
                    bad.append(f"{m.name}: column split {cr} does not tile [{rows}, {row_bytes}] bytes")
                if p is not None and storage_shape(p.dtype, p.shape) != (rows, row_bytes // DT_SIZE.get(p.dtype, 1)):
                    bad.append(f"{m.name}: column split rows {rows} x {row_bytes} B vs the parameter's {p.shape}")
        for pack, spans in by_pack.items():
            spans.sort()
            for a, b in zip(spans, spans[1:]):
                if b[0] < a[1]:
                    bad.append(f"{a[2]} and {b[2]} overlap in {pack}")
        if bad:
            raise ValueError(f"{role}: " + "; ".join(bad))

    def _banks(self, k: Kernel, buffers: dict, layer: int, kind: str) -> dict:
        """Layer `layer`'s parameters held by the bank inputs k_b<phase>_<name> [blocks, ...]."""
        out = {}
        phase, block = layer % 4, layer // 4
        for bank, param in BANKS[kind].items():
            name = f"k_b{phase}_{bank}"
            try:
                e = k.entry(name)
            except KeyError:
                continue
            t = buffers[name]
            per = e.bytes // e.shape[0]
            raw = _u8(t)[block * per:(block + 1) * per]
            out[param] = _typed(raw, e.dtype, e.shape[1:], e.name)
        for part in ("w_", "s_"):  # the GDN's q / k / v row blocks -> w_qkv / s_qkv
            parts = [out.pop(part + g, None) for g in ("gq", "gk", "gv")]
            if all(p is not None for p in parts):
                out[part + "qkv"] = torch.cat(parts, 0)
        return out

    def bind_layer(self, role: str, buffers: dict, layer: int) -> LayerParams:
        """Layer `layer` of the packed kernel `role` bound to the caller's buffers (device or host tensors keyed by
        the kernel's IO names: the packs, the banks and a MoE layer's experts e_gw<j> ..)."""
        k = self.kernel(role)
        kinds = k.kinds()
        if not 0 <= layer < len(kinds):
            raise ValueError(f"{role}: layer {layer} outside its {len(kinds)} layers")
        kind = kinds[layer]
        params = self.params.get(kind)
        if params is None:
            raise ValueError(f"manifest of {self.model}: no parameters of kind {kind!r}")
        phase = layer % 4
        inputs = {e.name for e in k.inputs}
        used = ({m.pack for m in k.layer_members(layer)} | {f"k_b{phase}_{b}" for b in BANKS[kind]}
                | {f"{b}{layer}" for b in EXPERT_IO}) & inputs
        k.check_buffers(buffers, names=used)
        w = {}
        for m in k.layer_members(layer):
            p = params.get(m.param)
            if p is None:
                raise ValueError(f"{m.name}: no parameter {m.param!r} of kind {kind}")
            raw = _u8(buffers[m.pack])[m.offset:m.offset + m.bytes]
            w[m.param] = _typed(m.to_row_major(raw).reshape(-1), p.dtype, p.shape, m.param)
        w.update(self._banks(k, buffers, layer, kind))
        for base in EXPERT_IO:  # a MoE layer's routed experts: IO e_gw<j> .. of the group (mkmanifest.py:326-336)
            name = f"{base}{layer}"
            if any(e.name == name for e in k.inputs):
                e = k.entry(name)
                w[base] = _typed(_u8(buffers[name]), e.dtype, e.shape, name)
        missing = [n for n in params if n not in w]
        if missing:
            raise ValueError(f"{role} layer {layer} ({kind}): parameters not found in packs or banks: {missing}")
        first = "qkv" if kind == "gdn" else "q"
        return LayerParams(kind, w, weight_format(params, first), weight_format(params, "gate"))

    def store_layer(self, role: str, buffers: dict, layer: int, weights: dict) -> None:
        """Writes a layer's parameters (axk.layer names, row-major) into the caller's packs and banks at the
        kernel's layout: the inverse of bind_layer, for a host that converts per-tensor weights into the pack format
        once (the reference's backend fills its packs the same way, q35_layer_pk.py:9-10)."""
        k = self.kernel(role)
        kind = k.kinds()[layer]
        params = self.params[kind]
        for m in k.layer_members(layer):
            p = params[m.param]
            src = _u8(weights[m.param].contiguous()).view(storage_shape(p.dtype, p.shape)[0], -1)
            _u8(buffers[m.pack])[m.offset:m.offset + m.bytes] = m.from_row_major(src)
        phase, block = layer % 4, layer // 4
        names = {e.name for e in k.inputs}
        for bank, param in BANKS[kind].items():
            name = f"k_b{phase}_{bank}"
            if name not in names:
                continue
            e = k.entry(name)
            per = e.bytes // e.shape[0]
            part = param[2:]
            if part in ("gq", "gk", "gv"):  # the q / k / v row blocks of w_qkv / s_qkv (q and k: KD rows each)
                full = weights[param[:2] + "qkv"]
                full = _u8(full.contiguous()).view(full.shape[0], -1)
                kd = k.entry(f"k_b{phase}_attn_w_q").shape[1]
                r0 = {"gq": 0, "gk": kd, "gv": 2 * kd}[part]
                src = full[r0:r0 + e.shape[1]].reshape(-1)
            else:
                src = _u8(weights[param].contiguous())
            _u8(buffers[name])[block * per:(block + 1) * per] = src


def gdn_conv_views(conv: torch.Tensor, num_k_heads: int, head_dim: int = 128) -> tuple:
    """The q / k / v column blocks (strided views) of a GDN conv state [B, K-1, 2 KD + VD]: the 9B group's resident
    cq<j> / ck<j> / cv<j> (models/qwen35_9b/whole/src/q35_group.py gdn_layer) over axk's one conv state."""
    kd = num_k_heads * head_dim
    return conv[..., :kd], conv[..., kd:2 * kd], conv[..., 2 * kd:]


def paged_cache_view(kv: torch.Tensor, num_kv_heads: int) -> torch.Tensor:
    """A group's resident paged cache kv<j> [P, 2, page, HKV D] as axk's [P, 2, page, HKV, D] (the same bytes)."""
    p, two, page, hd = kv.shape
    return kv.view(p, two, page, num_kv_heads, hd // num_kv_heads)


# ---- IO tables answered by libaxk (axk_io_table) --------------------------------------------------------------------
class _IoEntryC(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 48), ("bytes", ctypes.c_int64), ("dtype", ctypes.c_int32),
                ("output", ctypes.c_int32), ("rank", ctypes.c_int32), ("shape", ctypes.c_int64 * 6)]


ROLE_DIMS = {
    "lm_head": ("n", "k", "m"),
    "layer.gdn": ("hidden", "num_k_heads", "num_v_heads", "inter", "conv_kernel", "proj_fmt", "mlp_fmt",
                  "num_experts", "batch"),
    "layer.attn": ("hidden", "num_qo_heads", "num_kv_heads", "head_dim", "inter", "proj_fmt", "mlp_fmt",
                   "num_experts", "batch", "rot", "page_size", "num_pages"),
    "experts": ("num_experts", "hidden", "inter"),
}
_DEFAULTS = {"m": 1, "conv_kernel": 4, "proj_fmt": 2, "mlp_fmt": 2, "num_experts": 0, "batch": 1, "rot": 64,
             "page_size": 256, "num_pages": 1}


def io_table(role: str, **dims) -> dict:
    """The IO of `role` at `dims` as libaxk reports it: {"in": [[name, bytes, dtype, shape], ...], "out": [...]}.
    Formats may be given as "fp8" / "mxfp8" / "mxfp4"."""
    from .layer import WFMT

    if role not in ROLE_DIMS:
        raise ValueError(f"unknown role {role!r} (roles: {sorted(ROLE_DIMS)})")
    order = ROLE_DIMS[role]
    unknown = set(dims) - set(order)
    if unknown:
        raise ValueError(f"{role}: unknown dimensions {sorted(unknown)}")
    vals = []
    for n in order:
        v = dims.get(n, _DEFAULTS.get(n))
        if v is None:
            raise ValueError(f"{role}: dimension {n} is required")
        vals.append(WFMT[v] if isinstance(v, str) else int(v))
    arr = (ctypes.c_int64 * len(vals))(*vals)
    lib = _lib.load()
    count = ctypes.c_int(0)
    st = lib.axk_io_table(role.encode(), ctypes.addressof(arr), len(vals), None, 0, ctypes.addressof(count))
    if st not in (_lib.AXK_OK, 9):  # AXK_E_BUFFER: count holds the number of entries
        raise _lib.AxkError("axk_io_table", st, lib.axk_status_string(st).decode())
    buf = (_IoEntryC * max(1, count.value))()
    _lib.call("axk_io_table", role.encode(), ctypes.addressof(arr), len(vals), ctypes.addressof(buf), count.value,
              ctypes.addressof(count))
    out = {"in": [], "out": []}
    for e in buf[:count.value]:
        out["out" if e.output else "in"].append([e.name.decode(), int(e.bytes), int(e.dtype),
                                                 [int(e.shape[i]) for i in range(e.rank)]])
    return out
