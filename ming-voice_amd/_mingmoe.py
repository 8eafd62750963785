"""ctypes binding of libmingmoe.so (include/mingmoe.h) and the tensor plumbing the wrappers share.

The library is hand-written HIP for gfx950. It is loaded after torch, so its libamdhip64.so.7 dependency
binds to the HIP runtime torch already loaded (one runtime per process; streams and device pointers are
shared). There is no fallback: if the library is missing or a call fails, a RuntimeError says why.
"""
import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmingmoe.so")

MM_OK, MM_ERR_ARG, MM_ERR_HIP = 0, 1, 2
MM_BF16, MM_FP16, MM_FP32, MM_INT8, MM_INT32, MM_INT64 = range(6)
MM_SCORE_SIGMOID_GROUP, MM_SCORE_SOFTMAX = 0, 1
MM_PHASE_ALL, MM_PHASE_GATE_UP, MM_PHASE_DOWN, MM_PHASE_COMBINE = 0, 1, 2, 4
MM_NORM_ROUND_ONCE = 0x100
ABI_VERSION = 16

_DTYPES = {torch.bfloat16: MM_BF16, torch.float16: MM_FP16, torch.float32: MM_FP32, torch.int8: MM_INT8,
           torch.int32: MM_INT32, torch.int64: MM_INT64}

# exported entry points and their argument types (include/mingmoe.h)
_P, _I64, _I32, _F32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float


MM_PART_GATE, MM_PART_UP, MM_PART_DOWN = 0, 1, 2


class IngestItem(ctypes.Structure):
    """mm_ingest_item: one expert matrix in a file (path, absolute byte offset and size, dtype, where it goes)."""
    _fields_ = [("path", ctypes.c_char_p), ("offset", _I64), ("nbytes", _I64), ("src_dtype", ctypes.c_int32),
                ("part", ctypes.c_int32), ("slot", _I64), ("rows", _I64), ("cols", _I64)]


class Experts(ctypes.Structure):
    """mm_experts: stacked expert weights [E+1, 2I, H] / [E+1, H, I] (+ int8 row scales)."""
    _fields_ = [("w_gu", _P), ("w_d", _P), ("s_gu", _P), ("s_d", _P), ("w_dtype", ctypes.c_int32),
                ("s_dtype", ctypes.c_int32), ("n_slots", _I64), ("hidden", _I64), ("inter", _I64),
                ("gu_stride_e", _I64), ("gu_stride_n", _I64), ("d_stride_e", _I64), ("d_stride_n", _I64),
                ("sgu_stride_e", _I64), ("sd_stride_e", _I64), ("w_gu_slabs", _P), ("w_d_slabs", _P)]


SIGNATURES = {
    "mm_version": ([], ctypes.c_int),
    "mm_last_error": ([ctypes.c_char_p, ctypes.c_size_t], ctypes.c_size_t),
    "mm_rms_norm": ([_P, _I32, _I64, _I64, _I64, _P, _I32, _F32, _P, _I32, _I64, _P], ctypes.c_int),
    "mm_router": ([_P, _I32, _I64, _I64, _I64, _P, _I64, _P, _I32, _I32, _I32, _I32, _F32, _I32, _P, _P, _I32, _P,
                   _I64, _P], ctypes.c_int),
    "mm_router_select": ([_P, _I64, _I64, _P, _I32, _I32, _I32, _I32, _F32, _I32, _P, _I32, _P, _I64, _P],
                         ctypes.c_int),
    "mm_align_blocks": ([_P, _I32, _I64, ctypes.c_int32, ctypes.c_int32, _P, _P, _I64, _P, _P], ctypes.c_int),
    "mm_moe_decode": ([_P, _I64, _I64, ctypes.POINTER(Experts), _P, _I32, _I64, _I64, _P, _I64, _P, _I64, _P, _P,
                       _I64, _I32, _P], ctypes.c_int),
    "mm_moe_prefill": ([_P, _I64, _I64, ctypes.POINTER(Experts), _I64, _P, _I32, _P, _P, _P, _P, _I64,
                        ctypes.c_int32, _P, _I64, _P, _P, _P, _I64, _I32, _P], ctypes.c_int),
    "mm_moe_block_decode": ([_P, _I64, _I64, _P, _F32, _P, _I64, _P, _I32, _I32, _I32, _I32, _F32,
                             ctypes.POINTER(Experts), _P, _P, _I32, _P, _P, _P, _I32, _P, _I64, _P], ctypes.c_int),
    "mm_moe_block_decode_noalloc_bytes": ([_I64, _I64, _I64, _I64], ctypes.c_int64),
    "mm_moe_block_decode_noalloc": ([_P, _I64, _I64, _P, _F32, _P, _I64, _P, _I32, _I32, _I32, _I32, _F32,
                                     ctypes.POINTER(Experts), _P, _P, _I32, _P, _I32, _P, _I64, _P], ctypes.c_int),
    "mm_prefill_block_m": ([_I64, _I64, _I64, _I32], ctypes.c_int32),
    "mm_moe_block_prefill": ([_P, _I64, _I64, _P, _F32, _P, _I64, _P, _I32, _I32, _I32, _I32, _F32,
                              ctypes.POINTER(Experts), _P, _P, _I32, _P, _P, _P, _P, _P, _I64, _P, _P, _I32, _P,
                              _I64, _P], ctypes.c_int),
    "mm_small_linear": ([_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I32, _P, _I64, _P, _F32, _P, _P, _I64, _P],
                        ctypes.c_int),
    "mm_small_linear_glu": ([_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _F32, _P, _I64, _P], ctypes.c_int),
    "mm_quantize_rows_int8": ([_P, _I32, _I64, _I64, _I64, _P, _I64, _P, _I32, _P], ctypes.c_int),
    "mm_ingest_experts": ([ctypes.POINTER(IngestItem), _I64, ctypes.POINTER(Experts), _P, _P, _I64, _I32], ctypes.c_int),
    "mm_rope_attn": ([_P, _I64, _I64, _I64, _I32, _P, _P, _P, _P], ctypes.c_int),
    "mm_decode_attn_workspace": ([_I32, _I32, _I64], ctypes.c_int64),
    "mm_qwen_decode_attn": ([_P, _I32, _I32, _I32, _P, _P, _I64, _P, _I32, _P, _F32, _P, _P, _I64, _P],
                            ctypes.c_int),
    "mm_silu_mul": ([_P, _I64, _I64, _I64, _P, _I64, _P], ctypes.c_int),
    "mm_cfg_update": ([_P, _P, _I64, _I64, _F32, _P, _I32, _P, _P], ctypes.c_int),
    "mm_kda_recurrent": ([_P, _I64, _P, _I64, _P, _I64, _P, _I32, _I64, _P, _I32, _I64, _P, _P, _F32, _I32, _I32, _I32,
                          _F32, _I64, _I64, _I64, _I64, _P, _P, _I64, _P, _P, _I64, _P], ctypes.c_int),
    "mm_kda_recurrent_workspace": ([_I64, _I64, _I64], ctypes.c_int64),
    "mm_kda_chunk": ([_P, _I64, _P, _I64, _P, _I64, _P, _I32, _I64, _P, _I32, _I64, _P, _P, _F32, _I32, _I32, _I32,
                      _F32, _I64, _I64, _I64, _I64, _P, _P, _I64, _P, _P, _I64, _P], ctypes.c_int),
    "mm_kda_chunk_workspace": ([_I64, _I64, _I64], ctypes.c_int64),
    "mm_short_conv": ([_P, _I64, _I64, _I64, _P, _I64, _P, _P, _I32, _P, _I64, _P, _P], ctypes.c_int),
    "mm_short_conv_many": ([_I64, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I32, _P, _P], ctypes.c_int),
    "mm_rms_norm_gated": ([_P, _I64, _P, _I64, _P, _I64, _I64, _F32, _P, _I64, _P], ctypes.c_int),
    "mm_mla_attn_workspace": ([_I32, _I32, _I64], ctypes.c_int64),
    "mm_kda_decode_step": ([_P, _I64, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p), _I64, _P, _P,
                            _I64, _P, _P, _F32, _F32, _P, _I64, _I64, _I64, _P, _F32, _P, _P], ctypes.c_int),
    "mm_mla_decode_attn": ([_P, _P, _P, _I32, _I32, _I32, _P, _P, _I64, _P, _I32, _F32, _P, _P, _I64, _P], ctypes.c_int),
    "mm_mla_prefill_attn": ([_P, _I64, _P, _I64, _P, _I64, _I64, _I32, _I32, _I32, _P, _P, _I64, _P, _I32, _F32, _P,
                             _I64, _P], ctypes.c_int),
    "mm_embed_rows": ([_P, _I32, _I64, _I64, _I64, _P, _I32, _I64, _P, _I64, _P], ctypes.c_int),
    "mm_argmax_rows": ([_P, _I32, _I64, _I64, _I64, _P, _P], ctypes.c_int),
    "mm_argmax_rows_ws": ([_P, _I32, _I64, _I64, _I64, _P, _P, _I64, _P], ctypes.c_int),
    "mm_argmax_rows_workspace_bytes": ([_I64, _I64, _I32], ctypes.c_int64),
    "mm_gate_up_slabs_bytes": ([ctypes.POINTER(Experts)], _I64),
    "mm_gate_up_slabs": ([ctypes.POINTER(Experts), _P, _P], ctypes.c_int),
    "mm_down_slabs_bytes": ([ctypes.POINTER(Experts)], _I64),
    "mm_down_slabs": ([ctypes.POINTER(Experts), _P, _P], ctypes.c_int),
}

_lib = None


def load(path=LIB_PATH):
    """Loads (once) and returns the library with its argument types declared."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"libmingmoe.so not found at {path}: build it with `python build_lib.py` "
                           "(or __graft_entry__.build()); there is no fallback path")
    lib = ctypes.CDLL(path)
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    v = lib.mm_version()
    if v != ABI_VERSION:
        raise RuntimeError(f"libmingmoe.so ABI version {v}, expected {ABI_VERSION}: rebuild it")
    _lib = lib
    return lib


def last_error():
    lib = load()
    n = lib.mm_last_error(None, 0)
    buf = ctypes.create_string_buffer(int(n) + 1)
    lib.mm_last_error(buf, n + 1)
    return buf.value.decode(errors="replace")


def check(status, what):
    if status != MM_OK:
        msg = last_error()
        if status == MM_ERR_ARG:
            raise ValueError(f"{what}: {msg}")
        raise RuntimeError(f"{what}: {msg}")


def dtype_code(t):
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}") from None


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def stream_of(t):
    """Raw hipStream_t of torch's current stream on the tensor's device."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_gpu(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("libmingmoe kernels take GPU tensors only (got a tensor on "
                             f"{t.device}); there is no CPU path")
    dev = tensors[0].device
    for t in tensors[1:]:
        if t is not None and t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")


class on_device:
    """Makes the tensor's device current for the duration of a call (no-op when it already is)."""

    def __init__(self, t):
        self.dev = t.device.index

    def __enter__(self):
        self.prev = torch.cuda.current_device()
        if self.prev != self.dev:
            torch.cuda.set_device(self.dev)

    def __exit__(self, *exc):
        if self.prev != self.dev:
            torch.cuda.set_device(self.prev)
        return False


def version_of(t):
    """torch's in-place write counter of t (shared by every view of one base tensor), or None for tensors that keep
    none (made under torch.inference_mode)."""
    try:
        return t._version
    except RuntimeError:
        return None


def source_stamp(w):
    """What a prefill copy records of the stack it was made from: device, address, shape, strides and the write
    counter at the time of the copy. A copy is current for a stack while the stamps agree."""
    return (w.device.index, w.data_ptr(), tuple(w.shape), tuple(w.stride()), version_of(w))


def check_copy(copy, w, what):
    """Refuses (ValueError) a prefill copy that was not made from w by fused_moe.gate_up_slabs / down_slabs, or that
    w was written to since (torch's write counter moved: the loader's copy_ into the stack, an in-place op)."""
    stamp = getattr(copy, "_mm_source", None)
    if stamp is None:
        raise ValueError(f"{what} must be made by fused_moe.{'gate_up' if what == 'w_gu_slabs' else 'down'}_slabs "
                         "(it carries the stamp of its source stack)")
    now = source_stamp(w)
    if stamp[:4] != now[:4]:
        raise ValueError(f"{what} was made from another stack than the one passed")
    if stamp[4] is None or stamp[4] != now[4]:
        raise ValueError(f"{what} is stale: its stack was written to after the copy was made (make it again)")


def experts(w_gu, w_d, s_gu=None, s_d=None, w_gu_slabs=None, w_d_slabs=None):
    """mm_experts for stacked weights w_gu [E1, 2I, H], w_d [E1, H, I] (bf16 or int8 + scales); w_gu_slabs /
    w_d_slabs: the prefill copies of w_gu / w_d that fused_moe.gate_up_slabs / down_slabs make, or None. A copy that does not carry the current stamp of its stack is refused (check_copy)."""
    if w_gu.dim() != 3 or w_d.dim() != 3:
        raise ValueError("w_gu and w_d must be 3-D stacked expert tensors")
    E1, two_i, H = w_gu.shape
    I = w_d.shape[-1]
    if two_i != 2 * I or tuple(w_d.shape[:2]) != (E1, H):
        raise ValueError(f"inconsistent expert shapes w_gu {tuple(w_gu.shape)} w_d {tuple(w_d.shape)}")
    if w_gu.stride(2) != 1 or w_d.stride(2) != 1:
        raise ValueError("expert weights need a contiguous last dim")
    if w_gu.dtype != w_d.dtype or w_gu.dtype not in (torch.bfloat16, torch.int8):
        raise ValueError(f"expert weights must both be bf16 or int8 (got {w_gu.dtype}, {w_d.dtype})")
    q = w_gu.dtype == torch.int8
    if q != (s_gu is not None) or (s_gu is None) != (s_d is None):
        raise ValueError("int8 experts need s_gu and s_d; bf16 experts take none")
    ex = Experts()
    ex.w_gu, ex.w_d = w_gu.data_ptr(), w_d.data_ptr()
    ex.w_dtype = dtype_code(w_gu)
    ex.n_slots, ex.hidden, ex.inter = E1, H, I
    ex.gu_stride_e, ex.gu_stride_n = w_gu.stride(0), w_gu.stride(1)
    ex.d_stride_e, ex.d_stride_n = w_d.stride(0), w_d.stride(1)
    if q:
        if s_gu.dtype != s_d.dtype or s_gu.dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("int8 scales must both be fp32 or bf16")
        if tuple(s_gu.shape) != (E1, 2 * I) or tuple(s_d.shape) != (E1, H) or s_gu.stride(1) != 1 or s_d.stride(1) != 1:
            raise ValueError(f"scale shapes must be [E1, 2I] and [E1, H] (got {tuple(s_gu.shape)}, {tuple(s_d.shape)})")
        ex.s_gu, ex.s_d = s_gu.data_ptr(), s_d.data_ptr()
        ex.s_dtype = dtype_code(s_gu)
        ex.sgu_stride_e, ex.sd_stride_e = s_gu.stride(0), s_d.stride(0)
    else:
        ex.s_dtype = MM_FP32
    if w_gu_slabs is not None:
        if w_gu_slabs.dtype != w_gu.dtype or not w_gu_slabs.is_contiguous() or \
                w_gu_slabs.numel() != w_gu.shape[0] * w_gu.shape[1] * w_gu.shape[2] or w_gu_slabs.device != w_gu.device:
            raise ValueError("w_gu_slabs must be the contiguous prefill copy of w_gu (fused_moe.gate_up_slabs)")
        check_copy(w_gu_slabs, w_gu, "w_gu_slabs")
        ex.w_gu_slabs = w_gu_slabs.data_ptr()
    if w_d_slabs is not None:
        if w_d_slabs.dtype != w_d.dtype or not w_d_slabs.is_contiguous() or \
                w_d_slabs.numel() != w_d.shape[0] * w_d.shape[1] * w_d.shape[2] or w_d_slabs.device != w_d.device:
            raise ValueError("w_d_slabs must be the contiguous prefill copy of w_d (fused_moe.down_slabs)")
        check_copy(w_d_slabs, w_d, "w_d_slabs")
        ex.w_d_slabs = w_d_slabs.data_ptr()
    return ex
