"""Expert weights straight from safetensors shards into the stacked layout of the MoE kernels.

The reference builds the thinker on the GPU and streams each checkpoint tensor into its parameter
(direct_load.py:50-131); the MoE blocks pre-allocate their experts as views into stacked [E+1, 2I, H] /
[E+1, H, I] buffers (engine.py:150-188), and with int8 experts a per-tensor loader hook quantises each
expert matrix as it arrives (engine.py:126-147). Here one call per MoE block does that ingestion natively
(mm_ingest_experts): worker threads pread the expert matrices in file order into pinned staging, copy them
to the GPU on their own streams and land them in the stack, converting or quantising on the way.

  read_header(path)                      {key: (dtype, shape, begin, end)} of one .safetensors file
  checkpoint_index(model_dir)            {key: file path} from model.safetensors.index.json (or one file)
  expert_items(index, prefix, n_experts) the (key, part, slot) list of a MoE block's experts
  load_stacked_experts(...)              the block's stacked experts, bf16 or int8 + per-row scales
"""
import json
import os
import struct

import torch
from torch.autograd.graph import increment_version

import _mingmoe as _mm

__all__ = ["read_header", "checkpoint_index", "expert_items", "load_stacked_experts"]

_FILE_DTYPES = {"BF16": (_mm.MM_BF16, 2), "F16": (_mm.MM_FP16, 2), "F32": (_mm.MM_FP32, 4)}
_PARTS = (("gate_proj", _mm.MM_PART_GATE), ("up_proj", _mm.MM_PART_UP), ("down_proj", _mm.MM_PART_DOWN))


def read_header(path):
    """The tensor table of a .safetensors file: an 8-byte little-endian header size, then a JSON object of
    {key: {"dtype", "shape", "data_offsets": [begin, end]}} with offsets relative to the end of the header
    (the format direct_load.py:24-29 reads). Returns {key: (dtype, shape, abs_begin, abs_end)}."""
    with open(path, "rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise ValueError(f"{path}: not a safetensors file (no header size)")
        n = struct.unpack("<Q", raw)[0]
        meta = json.loads(f.read(n))
    base = 8 + n
    out = {}
    for k, info in meta.items():
        if k == "__metadata__":
            continue
        a, b = info["data_offsets"]
        out[k] = (info["dtype"], tuple(info["shape"]), base + a, base + b)
    return out


def checkpoint_index(model_dir):
    """{key: absolute file path} of a checkpoint directory (model.safetensors.index.json, as
    direct_load.py:80 reads it, or a single model.safetensors)."""
    idx = os.path.join(model_dir, "model.safetensors.index.json")
    if os.path.exists(idx):
        with open(idx) as f:
            wm = json.load(f)["weight_map"]
        return {k: os.path.join(model_dir, v) for k, v in wm.items()}
    one = os.path.join(model_dir, "model.safetensors")
    if not os.path.exists(one):
        raise FileNotFoundError(f"{model_dir}: neither model.safetensors.index.json nor model.safetensors")
    return {k: one for k in read_header(one)}


def expert_items(index, prefix, n_experts, shared=True):
    """(key, part, slot) for the routed experts 0..n_experts-1 of the MoE block `prefix` (keys
    `{prefix}.experts.{e}.{gate,up,down}_proj.weight`, engine.py:139-143) and, with `shared`, its shared
    expert (`{prefix}.shared_experts.*`) in slot n_experts (engine.py:345-361)."""
    out = []
    for e in range(n_experts):
        for name, part in _PARTS:
            out.append((f"{prefix}.experts.{e}.{name}.weight", part, e))
    if shared:
        for name, part in _PARTS:
            out.append((f"{prefix}.shared_experts.{name}.weight", part, n_experts))
    missing = [k for k, _, _ in out if k not in index]
    if missing:
        raise ValueError(f"{len(missing)} expert tensors missing from the checkpoint, e.g. {missing[:3]}")
    return out


def load_stacked_experts(index, prefix, n_experts, *, shared=True, int8=False, scale_dtype=torch.float32,
                         device="cuda", out=None, threads=4):
    """Reads the MoE block `prefix`'s experts from the checkpoint `index` ({key: file}, or a model directory)
    into stacked tensors on `device`: {"w_gu": [E1, 2I, H], "w_d": [E1, H, I]} in bf16, or with int8=True
    {"q_gu", "q_d" (int8), "s_gu": [E1, 2I], "s_d": [E1, H] (scale_dtype)}, E1 = n_experts + 1 with the shared
    expert. `out` may hold those tensors already (for example the views a model's MoE block owns); they are
    filled in place. int8 rows are quantised as quantize_rows_int8 does; fp16 / fp32 file data is rounded
    to bf16. Blocks until the stack is complete. `threads` readers (4 measured best on MI355X: 53-54 GB/s of
    page-cached file data, 93 % of the pinned host-to-device copy rate)."""
    if isinstance(index, (str, os.PathLike)):
        index = checkpoint_index(index)
    items = expert_items(index, prefix, n_experts, shared)
    headers = {}
    rows = []
    for key, part, slot in items:
        path = index[key]
        if path not in headers:
            headers[path] = read_header(path)
        dt, shape, a, b = headers[path][key]
        if dt not in _FILE_DTYPES:
            raise ValueError(f"{key}: file dtype {dt} is not one of {sorted(_FILE_DTYPES)}")
        if len(shape) != 2:
            raise ValueError(f"{key}: expected a matrix, got shape {shape}")
        rows.append((path, a, b - a, _FILE_DTYPES[dt][0], part, slot, shape[0], shape[1]))
    I, H = next(r[6:8] for r in rows if r[4] == _mm.MM_PART_GATE)
    E1 = n_experts + (1 if shared else 0)
    dev = torch.device(device)
    if out is None:
        if int8:
            out = {"q_gu": torch.empty(E1, 2 * I, H, dtype=torch.int8, device=dev),
                   "q_d": torch.empty(E1, H, I, dtype=torch.int8, device=dev),
                   "s_gu": torch.empty(E1, 2 * I, dtype=scale_dtype, device=dev),
                   "s_d": torch.empty(E1, H, dtype=scale_dtype, device=dev)}
        else:
            out = {"w_gu": torch.empty(E1, 2 * I, H, dtype=torch.bfloat16, device=dev),
                   "w_d": torch.empty(E1, H, I, dtype=torch.bfloat16, device=dev)}
    _mm.require_gpu(*out.values())
    if int8:
        ex = _mm.experts(out["q_gu"], out["q_d"], out["s_gu"], out["s_d"])
    else:
        ex = _mm.experts(out["w_gu"], out["w_d"])
    if ex.inter != I or ex.hidden != H:
        raise ValueError(f"the stack holds I={ex.inter}, H={ex.hidden}; the checkpoint has I={I}, H={H}")
    arr = (_mm.IngestItem * len(rows))()
    paths = [p.encode() for p, *_ in rows]  # keep the bytes alive for the call
    for i, (r, pb) in enumerate(zip(rows, paths)):
        _, off, nbytes, sdt, part, slot, nr, nc = r
        arr[i] = _mm.IngestItem(pb, off, nbytes, sdt, part, slot, nr, nc)
    slot_bytes = max(r[2] for r in rows)
    slot_bytes = (slot_bytes + 4095) // 4096 * 4096
    threads = max(1, min(int(threads), len(rows)))
    host = torch.empty(2 * threads * slot_bytes, dtype=torch.uint8, pin_memory=True)
    stage = torch.empty(threads * slot_bytes, dtype=torch.uint8, device=dev)
    lib = _mm.load()
    with _mm.on_device(stage):
        torch.cuda.current_stream(dev).synchronize()  # allocation and any earlier writes to the stack are done
        _mm.check(lib.mm_ingest_experts(arr, len(rows), ex, _mm.ptr(host), _mm.ptr(stage), slot_bytes, threads),
                  "load_stacked_experts")
    # the library wrote the stacks through raw pointers, which torch's write counters do not see: move them, so
    # that a prefill copy made before this load counts as stale (fused_moe.prefill_copies)
    for t in out.values():
        if _mm.version_of(t) is not None:
            increment_version(t)
    return out
