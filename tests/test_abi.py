"""CPU checks of the C ABI: the library loads and exports every entry point of include/mingmoe.h, the
ctypes struct matches the C layout, and argument validation fails with a message before any GPU work."""
import ctypes
import os
import re
import subprocess

import pytest
import torch

import _mingmoe as mm

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mingmoe.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|int32_t|int64_t|size_t)\s+(mm_\w+)\s*\(", text, re.M)))


def test_header_declares_the_expected_entry_points():
    assert _declared() == sorted(mm.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = mm.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.mm_version() == mm.ABI_VERSION


def test_experts_struct_layout_matches_c(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "mingmoe.h"\n'
                   'int main(void){printf("%zu", sizeof(mm_experts));'
                   + "".join(f'printf(" %zu", offsetof(mm_experts, {f}));' for f, _ in mm.Experts._fields_)
                   + 'return 0;}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)], check=True)
    vals = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert vals[0] == ctypes.sizeof(mm.Experts)
    assert vals[1:] == [getattr(mm.Experts, f).offset for f, _ in mm.Experts._fields_]


def _err(rc):
    assert rc == mm.MM_ERR_ARG
    return mm.last_error()


def test_argument_validation_reports_messages():
    lib = mm.load()
    P = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation first
    assert "bad shape" in _err(lib.mm_rms_norm(P, mm.MM_BF16, -1, 64, 64, P, mm.MM_BF16, 1e-6, P, mm.MM_BF16, 64, None))
    assert "top_k" in _err(lib.mm_router(P, mm.MM_BF16, 1, 64, 64, P, 64, None, mm.MM_SCORE_SOFTMAX, 1, 1, 65, 1.0, 1,
                                         P, P, mm.MM_INT64, P, 66, None))
    assert "n_group" in _err(lib.mm_router(P, mm.MM_BF16, 1, 64, 64, P, 64, None, mm.MM_SCORE_SOFTMAX, 2, 1, 6, 1.0, 1,
                                           P, P, mm.MM_INT64, P, 7, None))
    assert "nb=" in _err(lib.mm_align_blocks(P, mm.MM_INT64, 100, 65, 64, P, P, 3, None, None))
    assert "n_slots" in _err(lib.mm_align_blocks(P, mm.MM_INT64, 100, 300, 64, P, P, 400, None, None))
    assert "null expert descriptor" in _err(lib.mm_moe_decode(P, 1, 64, None, P, mm.MM_INT64, 7, 7, P, 7, None, 0, P,
                                                              P, 64, 0, None))
    ex = mm.Experts()
    ex.w_gu, ex.w_d, ex.w_dtype, ex.n_slots, ex.hidden, ex.inter = 16, 16, mm.MM_BF16, 65, 2048, 1408
    ex.gu_stride_e, ex.gu_stride_n, ex.d_stride_e, ex.d_stride_n = 2816 * 2048, 2048, 2048 * 1408, 1408
    assert "n_tokens * nk" in _err(lib.mm_moe_decode(P, 10, 2048, ctypes.byref(ex), P, mm.MM_INT64, 7, 7, P, 7, None,
                                                     0, P, P, 2048, 0, None))
    ex.w_gu = 18  # misaligned rows
    assert "16-byte aligned" in _err(lib.mm_moe_decode(P, 1, 2048, ctypes.byref(ex), P, mm.MM_INT64, 7, 7, P, 7, None,
                                                       0, P, P, 2048, 0, None))
    ex.w_gu, ex.hidden = 16, 2047
    assert "multiples" in _err(lib.mm_moe_prefill(P, 4, 2048, ctypes.byref(ex), 7, P, mm.MM_INT64, P, P, P, P, 10,
                                                  64, None, 0, P, P, P, 2048, 0, None))
    ex.hidden = 2048
    assert "block_m" in _err(lib.mm_moe_prefill(P, 4, 2048, ctypes.byref(ex), 7, P, mm.MM_INT64, P, P, P, P, 10,
                                                32, None, 0, P, P, P, 2048, 0, None))
    assert "M=17" in _err(lib.mm_small_linear(P, 17, 64, 64, P, 64, 64, None, 0, None, 0, None, 0.0, None, P, 64, None))
    assert "scale dtype" in _err(lib.mm_quantize_rows_int8(P, mm.MM_BF16, 4, 64, 64, P, 64, P, mm.MM_INT8, None))
    assert "seq=9" in _err(lib.mm_rope_attn(P, 2, 9, 1024, 16, P, P, P, None))
    arrP, arr64 = (ctypes.c_void_p * 4)(16, 16, 16, 16), (ctypes.c_int64 * 4)(64, 64, 64, 64)
    assert "convolutions (1 to 4)" in _err(lib.mm_short_conv_many(5, arrP, arr64, arr64, arrP, arrP, arrP, arr64, 8, 4,
                                                                  1, None, None))
    assert "kernel width" in _err(lib.mm_short_conv_many(3, arrP, arr64, arr64, arrP, arrP, arrP, arr64, 8, 9, 1, None,
                                                         None))
    bad_c = (ctypes.c_int64 * 4)(64, 0, 64, 64)
    assert "bad C=0 (convolution 1)" in _err(lib.mm_short_conv_many(3, arrP, arr64, bad_c, arrP, arrP, arrP, arr64, 8,
                                                                    4, 1, None, None))
    assert "null array" in _err(lib.mm_short_conv_many(3, None, arr64, arr64, arrP, arrP, arrP, arr64, 8, 4, 1, None,
                                                       None))
    assert "head dim 65" in _err(lib.mm_rope_attn(P, 2, 3, 1040, 16, P, P, P, None))
    assert "head dim 48" in _err(lib.mm_qwen_decode_attn(P, 8, 2, 48, P, P, 64, P, mm.MM_INT64, P, 0.1, P, P, 1 << 20,
                                                         None))
    assert "at most 16" in _err(lib.mm_qwen_decode_attn(P, 34, 2, 64, P, P, 64, P, mm.MM_INT64, P, 0.1, P, P, 1 << 20,
                                                        None))
    assert lib.mm_prefill_block_m(2048, 7, 65, mm.MM_BF16) == 128 and lib.mm_prefill_block_m(512, 7, 65, mm.MM_BF16) == 64
    assert lib.mm_prefill_block_m(2048, 7, 65, mm.MM_INT8) == 64 and lib.mm_prefill_block_m(1189, 7, 65, mm.MM_BF16) == 128
    assert lib.mm_prefill_block_m(1188, 7, 65, mm.MM_BF16) == 64
    need = lib.mm_decode_attn_workspace(14, 64, 1024)
    assert need == 14 * 16 * (64 + 2) * 4 and lib.mm_decode_attn_workspace(0, 64, 1024) == 0
    assert "workspace needs" in _err(lib.mm_qwen_decode_attn(P, 14, 2, 64, P, P, 1024, P, mm.MM_INT64, P, 0.1, P, P,
                                                             need - 4, None))
    assert "int32 or int64" in _err(lib.mm_qwen_decode_attn(P, 14, 2, 64, P, P, 1024, P, mm.MM_FP32, P, 0.1, P, P,
                                                            need, None))
    assert "row stride" in _err(lib.mm_silu_mul(P, 1, 4864, 4864, P, 4864, None))
    assert "up to 8192" in _err(lib.mm_small_linear_glu(P, 1, 9216, 9216, P, 64, 9216, None, 0.0, P, 64, None))
    ex = mm.Experts()
    ex.w_gu, ex.w_d, ex.w_dtype, ex.n_slots, ex.hidden, ex.inter = 16, 16, mm.MM_BF16, 5, 256, 128
    ex.gu_stride_e, ex.gu_stride_n, ex.d_stride_e, ex.d_stride_n = 256 * 256, 256, 256 * 128, 128
    items = (mm.IngestItem * 1)(mm.IngestItem(b"/nonexistent", 0, 128 * 256 * 2, mm.MM_BF16, mm.MM_PART_DOWN, 0,
                                              128, 256))
    assert "does not fit the stack" in _err(lib.mm_ingest_experts(items, 1, ctypes.byref(ex), P, P, 1 << 20, 2))
    items[0] = mm.IngestItem(b"/nonexistent", 0, 1000, mm.MM_BF16, mm.MM_PART_GATE, 0, 128, 256)
    assert "bytes for a" in _err(lib.mm_ingest_experts(items, 1, ctypes.byref(ex), P, P, 1 << 20, 2))
    items[0] = mm.IngestItem(b"/nonexistent", 0, 128 * 256 * 2, mm.MM_BF16, mm.MM_PART_GATE, 5, 128, 256)
    assert "slot 5" in _err(lib.mm_ingest_experts(items, 1, ctypes.byref(ex), P, P, 1 << 20, 2))
    ex.w_dtype = mm.MM_INT8
    assert "needs fp32 or bf16 scales" in _err(lib.mm_ingest_experts(items, 1, ctypes.byref(ex), P, P, 1 << 20, 2))
    assert "bf16 or fp32" in _err(lib.mm_argmax_rows(P, mm.MM_INT8, 1, 64, 64, P, None))
    assert "n=0" in _err(lib.mm_argmax_rows(P, mm.MM_BF16, 1, 0, 64, P, None))
    assert "row stride" in _err(lib.mm_argmax_rows(P, mm.MM_FP32, 2, 64, 32, P, None))
    assert lib.mm_argmax_rows_workspace_bytes(1, 126464, mm.MM_BF16) == 31 * 8
    assert lib.mm_argmax_rows_workspace_bytes(1, 0, mm.MM_BF16) == -1
    assert "workspace of 8 bytes" in _err(lib.mm_argmax_rows_ws(P, mm.MM_BF16, 1, 126464, 126464, P, P, 8, None))
    assert "null pointer" in _err(lib.mm_argmax_rows_ws(P, mm.MM_BF16, 1, 126464, 126464, P, None, 1024, None))
    assert "int32 or int64" in _err(lib.mm_embed_rows(P, mm.MM_BF16, 100, 64, 64, P, mm.MM_FP32, 1, P, 64, None))
    assert "16-byte aligned" in _err(lib.mm_embed_rows(P, mm.MM_BF16, 100, 12, 12, P, mm.MM_INT64, 1, P, 12, None))
    assert "bf16, fp16 or fp32" in _err(lib.mm_embed_rows(P, mm.MM_INT8, 100, 64, 64, P, mm.MM_INT64, 1, P, 64, None))
    ex = mm.Experts()
    ex.w_gu, ex.w_d, ex.w_dtype, ex.n_slots, ex.hidden, ex.inter = 16, 16, mm.MM_BF16, 65, 2048, 1408
    ex.gu_stride_e, ex.gu_stride_n, ex.d_stride_e, ex.d_stride_n = 2816 * 2048, 2048, 2048 * 1408, 1408
    assert lib.mm_gate_up_slabs_bytes(ctypes.byref(ex)) == 65 * 2816 * 2048 * 2
    ex.w_gu_slabs = 24  # misaligned copy
    assert "must be 16-byte aligned" in _err(lib.mm_moe_prefill(P, 4, 2048, ctypes.byref(ex), 7, P, mm.MM_INT64, P, P,
                                                                P, P, 10, 64, None, 0, P, P, P, 2048, 0, None))
    assert "out must be" in _err(lib.mm_gate_up_slabs(ctypes.byref(ex), ctypes.c_void_p(8), None))
    ex.hidden, ex.gu_stride_n, ex.gu_stride_e, ex.d_stride_e = 2040, 2040, 2816 * 2040, 2040 * 1408
    assert lib.mm_gate_up_slabs_bytes(ctypes.byref(ex)) == 0
    assert "hidden a multiple of 64" in _err(lib.mm_gate_up_slabs(ctypes.byref(ex), P, None))
    ex.hidden, ex.gu_stride_n, ex.gu_stride_e, ex.d_stride_e = 2048, 2048, 2816 * 2048, 2048 * 1408
    ex.w_dtype, ex.s_gu, ex.s_d, ex.s_dtype, ex.sgu_stride_e, ex.sd_stride_e = mm.MM_INT8, 16, 16, mm.MM_FP32, 2816, 2048
    ex.w_gu_slabs = 32
    assert lib.mm_gate_up_slabs_bytes(ctypes.byref(ex)) == 65 * 2816 * 2048  # int8 copies: 16-row pieces, 1 byte each
    ex.hidden, ex.gu_stride_n, ex.gu_stride_e, ex.d_stride_e = 2064, 2064, 2816 * 2064, 2064 * 1408  # 16 x 129
    ex.sd_stride_e = 2064
    assert lib.mm_gate_up_slabs_bytes(ctypes.byref(ex)) == 0
    assert "needs hidden a multiple of 64" in _err(lib.mm_moe_prefill(
        P, 4, 2064, ctypes.byref(ex), 7, P, mm.MM_INT64, P, P, P, P, 10, 64, None, 0, P, P, P, 2064, 0, None))
    assert "or 16 (int8)" in _err(lib.mm_gate_up_slabs(ctypes.byref(ex), P, None))
    # the prefill copy of w_d
    ex = mm.Experts()
    ex.w_gu, ex.w_d, ex.w_dtype, ex.n_slots, ex.hidden, ex.inter = 16, 16, mm.MM_BF16, 65, 2048, 1408
    ex.gu_stride_e, ex.gu_stride_n, ex.d_stride_e, ex.d_stride_n = 2816 * 2048, 2048, 2048 * 1408, 1408
    assert lib.mm_down_slabs_bytes(ctypes.byref(ex)) == 65 * 2048 * 1408 * 2
    ex.w_d_slabs = 24  # misaligned copy
    assert "prefill copy of w_d must be 16-byte aligned" in _err(lib.mm_moe_prefill(
        P, 4, 2048, ctypes.byref(ex), 7, P, mm.MM_INT64, P, P, P, P, 10, 64, None, 0, P, P, P, 2048, 0, None))
    assert "out must be" in _err(lib.mm_down_slabs(ctypes.byref(ex), ctypes.c_void_p(8), None))
    ex.inter, ex.gu_stride_e, ex.d_stride_e, ex.d_stride_n = 1400, 2800 * 2048, 2048 * 1400, 1400
    assert lib.mm_down_slabs_bytes(ctypes.byref(ex)) == 0
    assert "inter a multiple of 64" in _err(lib.mm_down_slabs(ctypes.byref(ex), P, None))
    ex.w_d_slabs = 32
    assert "a prefill copy of w_d needs inter a multiple of 64" in _err(lib.mm_moe_prefill(
        P, 4, 2048, ctypes.byref(ex), 7, P, mm.MM_INT64, P, P, P, P, 10, 64, None, 0, P, P, P, 2048, 0, None))
    ex.inter, ex.gu_stride_e, ex.d_stride_e, ex.d_stride_n = 1408, 2816 * 2048, 2048 * 1408, 1408
    ex.w_dtype, ex.s_gu, ex.s_d, ex.s_dtype, ex.sgu_stride_e, ex.sd_stride_e = mm.MM_INT8, 16, 16, mm.MM_FP32, 2816, 2048
    assert lib.mm_down_slabs_bytes(ctypes.byref(ex)) == 65 * 2048 * 1408
    ex.hidden, ex.sd_stride_e, ex.d_stride_e, ex.gu_stride_n, ex.gu_stride_e = 2056, 2056, 2056 * 1408, 2056, 2816 * 2056
    assert lib.mm_down_slabs_bytes(ctypes.byref(ex)) == 0  # hidden 2056: a multiple of 8, not of 16


def test_wrappers_refuse_cpu_tensors():
    import fused_moe
    import fused_ops
    import fastlinear
    x = torch.zeros(1, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="no CPU path"):
        fused_ops.rms_norm(x, torch.ones(64, dtype=torch.bfloat16), 1e-6)
    with pytest.raises(ValueError, match="no CPU path"):
        fused_moe.quantize_rows_int8(x)
    with pytest.raises(ValueError, match="no CPU path"):
        fastlinear.small_linear(x, torch.zeros(8, 64, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="no CPU path"):
        fused_moe._align_blocks(torch.zeros(7, dtype=torch.long), 65, 64)
    with pytest.raises(ValueError, match="no CPU path"):
        fused_moe.gate_up_slabs(torch.zeros(1, 8, 64, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="no CPU path"):
        fused_moe.down_slabs(torch.zeros(1, 8, 64, dtype=torch.bfloat16))
    import fast_talker
    with pytest.raises(ValueError, match="no CPU path"):
        fast_talker.silu_mul(torch.zeros(1, 64, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="no CPU path"):
        fast_talker.rope_attn(torch.zeros(1, 3, 192, dtype=torch.bfloat16), torch.ones(3, 16), torch.zeros(3, 16), 2)


def test_reference_module_surface_is_kept():
    import fast_talker
    import fused_moe
    import fused_ops
    import fastlinear
    for mod, names in ((fused_moe, ["fused_moe_decode", "fused_moe_prefill", "quantize_rows_int8", "_align_blocks",
                                    "CFG", "GCFG", "_graph_us"]),
                       (fused_ops, ["rms_norm", "moe_route"]),
                       (fastlinear, ["small_linear", "save_cache", "_graph_time", "CACHE_FILE", "_best"]),
                       (fast_talker, ["rope_attn", "_fuse", "_Block", "_rope_tables", "FastTail", "FastQwen2Step",
                                      "qwen_decode_attn", "silu_mul"])):
        for n in names:
            assert hasattr(mod, n), f"{mod.__name__}.{n}"
    fastlinear.save_cache()  # nothing tuned: writes nothing


def test_decode_refuses_expert_spans_beyond_32_bit_offsets():
    """The decode kernels read one expert's rows through a buffer resource addressed by 32-bit offsets, with
    2^31 as the offset that reads zero; a descriptor whose expert spans 2^31 bytes or more is refused before any
    launch (an int8 expert with 2 x 32768 gate/up rows of 32768 bytes spans exactly 2^31)."""
    lib = mm.load()
    P = ctypes.c_void_p(16)
    ex = mm.Experts()
    ex.w_gu, ex.w_d, ex.s_gu, ex.s_d, ex.w_dtype, ex.s_dtype = 16, 16, 16, 16, mm.MM_INT8, mm.MM_FP32
    ex.n_slots, ex.hidden, ex.inter = 2, 32768, 32768
    ex.gu_stride_n, ex.d_stride_n = 32768, 32768
    ex.gu_stride_e, ex.d_stride_e = 2 * 32768 * 32768, 32768 * 32768
    ex.sgu_stride_e, ex.sd_stride_e = 2 * 32768, 32768
    assert "2^31" in _err(lib.mm_moe_decode(P, 1, 32768, ctypes.byref(ex), P, mm.MM_INT64, 7, 7, P, 7, None, 0, P, P,
                                            32768, 0, None))
    ex.inter = 16384  # 2 x 16384 rows of 32768 bytes = 2^30: passes this check and stops at the next (10 x 7 pairs)
    ex.gu_stride_e, ex.d_stride_e, ex.sgu_stride_e = 2 * 16384 * 32768, 32768 * 16384, 2 * 16384
    ex.d_stride_n = 16384
    assert "n_tokens * nk" in _err(lib.mm_moe_decode(P, 10, 32768, ctypes.byref(ex), P, mm.MM_INT64, 7, 7, P, 7, None,
                                                     0, P, P, 32768, 0, None))


def test_kda_chunk_workspace_and_argument_checks():
    """mm_kda_chunk_workspace: one block of 49 K + 512 floats per (16-token chunk, head); mm_kda_chunk refuses a
    short workspace before any launch, naming itself."""
    lib = mm.load()
    assert lib.mm_kda_chunk_workspace(2, 16, 128) == 0 == lib.mm_kda_recurrent_workspace(2, 16, 128)
    assert lib.mm_kda_chunk_workspace(5, 16, 96) == -1
    for T, H, K in ((512, 16, 128), (17, 3, 64), (3, 1, 128)):
        rows = T * H * (3 * K + 4) * 4
        assert lib.mm_kda_recurrent_workspace(T, H, K) == rows
        assert lib.mm_kda_chunk_workspace(T, H, K) == (T + 15) // 16 * H * (49 * K + 512) * 4
    rc = lib.mm_kda_chunk(16, 2048, 16, 2048, 16, 2048, 16, mm.MM_FP32, 2048, 16, mm.MM_FP32, 16, None, None,
                          float("nan"), 1, 0, 0, 1.0, 40, 16, 128, 128, 16, 16, 2048, None, 16,
                          lib.mm_kda_chunk_workspace(40, 16, 128) - 16, None)
    assert rc == mm.MM_ERR_ARG and "kda_chunk" in mm.last_error() and "workspace" in mm.last_error()
    with pytest.raises(ValueError, match="no CPU path"):
        import thinker_attn
        z = torch.zeros(1, 4, 2, 64, dtype=torch.bfloat16)
        thinker_attn.chunk_kda(z, z, z, z, torch.zeros(1, 4, 2))
