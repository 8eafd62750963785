"""GPU parity of the expert ingestion (mm_ingest_experts) against the reference's restacking and the
oracle's quantiser: the stacks must be bit-exact (a copy, a round-to-nearest-even cast, an integer code)."""
import pytest
import torch

import expert_load as EL
from ckpt_util import stacked
from workloads import expert_tensors, write_checkpoint
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
PFX = "model.layers.2.mlp"


@pytest.fixture(scope="module")
def ck(tmp_path_factory):
    t = expert_tensors(PFX, 6, 256, 128, seed=5)
    return t, write_checkpoint(str(tmp_path_factory.mktemp("ck")), t, shards=3)


@pytest.mark.parametrize("threads", [1, 3, 8])
def test_bf16_stack_is_the_checkpoint(ck, threads):
    t, root = ck
    print(f"ingest bf16 threads={threads}", flush=True)
    out = EL.load_stacked_experts(root, PFX, 6, threads=threads)
    torch.cuda.synchronize()
    w_gu, w_d = stacked(t, PFX, 6)
    assert torch.equal(out["w_gu"].cpu(), w_gu) and torch.equal(out["w_d"].cpu(), w_d)


@pytest.mark.parametrize("sdt", [torch.float32, torch.bfloat16])
def test_int8_stack_matches_the_quantiser(ck, sdt):
    t, root = ck
    print(f"ingest int8 scales={sdt}", flush=True)
    out = EL.load_stacked_experts(root, PFX, 6, int8=True, scale_dtype=sdt)
    torch.cuda.synchronize()
    w_gu, w_d = stacked(t, PFX, 6)
    for w, q, s in ((w_gu, out["q_gu"], out["s_gu"]), (w_d, out["q_d"], out["s_d"])):
        qo, so = O.quantize_rows_int8(w, scale_dtype=sdt)
        assert torch.equal(q.cpu(), qo) and torch.equal(s.cpu(), so)


@pytest.mark.parametrize("fdt", [torch.float32, torch.float16])
def test_wide_file_dtypes_round_to_bf16(tmp_path, fdt):
    t = expert_tensors(PFX, 3, 128, 64, seed=6, dtype=torch.float32)
    t = {k: v.to(fdt) for k, v in t.items()}
    root = write_checkpoint(str(tmp_path / "ck"), t, shards=2)
    out = EL.load_stacked_experts(root, PFX, 3, threads=2)
    q = EL.load_stacked_experts(root, PFX, 3, int8=True, scale_dtype=torch.float32, threads=2)
    torch.cuda.synchronize()
    w_gu, w_d = stacked(t, PFX, 3)
    assert torch.equal(out["w_gu"].cpu(), w_gu.to(torch.bfloat16)) and torch.equal(out["w_d"].cpu(), w_d.to(torch.bfloat16))
    qo, so = O.quantize_rows_int8(w_gu.float())  # the quantiser reads the file's own precision
    assert torch.equal(q["q_gu"].cpu(), qo) and torch.equal(q["s_gu"].cpu(), so)


def test_thinker_shape_into_prestacked_views(tmp_path):
    """Hidden 2048, intermediate 1408 (the benchmarked block), 4 routed experts + shared, loaded in place into
    views of larger buffers the way a model's MoE block owns its stack."""
    t = expert_tensors(PFX, 4, 2048, 1408, seed=7)
    root = write_checkpoint(str(tmp_path / "ck"), t, shards=2)
    big_gu = torch.zeros(7, 2816, 2048, dtype=torch.bfloat16, device=DEV)
    big_d = torch.zeros(7, 2048, 1408, dtype=torch.bfloat16, device=DEV)
    out = {"w_gu": big_gu[1:6], "w_d": big_d[1:6]}
    EL.load_stacked_experts(root, PFX, 4, out=out, threads=4)
    torch.cuda.synchronize()
    w_gu, w_d = stacked(t, PFX, 4)
    assert torch.equal(big_gu[1:6].cpu(), w_gu) and torch.equal(big_d[1:6].cpu(), w_d)
    assert not big_gu[0].any() and not big_gu[6].any() and not big_d[0].any() and not big_d[6].any()


def test_shape_mismatch_is_refused(ck):
    _, root = ck
    out = {"w_gu": torch.empty(7, 2 * 64, 256, dtype=torch.bfloat16, device=DEV),
           "w_d": torch.empty(7, 256, 64, dtype=torch.bfloat16, device=DEV)}
    with pytest.raises(ValueError, match="I=64"):
        EL.load_stacked_experts(root, PFX, 6, out=out)
