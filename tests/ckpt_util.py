"""The reference's restacking of checkpoint expert tensors (engine.py:343-361), as a check for the ingestion
tests; the synthetic checkpoints themselves come from workloads.expert_tensors / write_checkpoint."""
import torch


def stacked(tensors, prefix, n_experts):
    """The reference restacking (engine.py:343-361) on the CPU: w_gu [E1, 2I, H], w_d [E1, H, I]."""
    gu, d = [], []
    for e in list(range(n_experts)) + ["shared"]:
        p = f"{prefix}.shared_experts." if e == "shared" else f"{prefix}.experts.{e}."
        gu.append(torch.cat([tensors[p + "gate_proj.weight"], tensors[p + "up_proj.weight"]]))
        d.append(tensors[p + "down_proj.weight"])
    return torch.stack(gu), torch.stack(d)
