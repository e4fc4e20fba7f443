"""Host checks of axk.DecodeGroup (no GPU): the group's argument contract is enforced before anything is
allocated or launched."""
import pytest
import torch

from axk import group


def test_group_rejects_bad_layers():
    with pytest.raises(ValueError, match="at least one layer"):
        group.DecodeGroup([], 1, 64, "cpu")
    with pytest.raises(ValueError, match="kinds"):
        group.DecodeGroup([{"kind": "x", "w": {}}], 1, 64, "cpu")
    with pytest.raises(ValueError, match="page table"):
        group.DecodeGroup([{"kind": "a", "w": {}}], 1, 64, "cpu", num_qo_heads=2, rot=64)
    attn = {k: torch.zeros(1) for k in ("cos", "sin", "indptr", "indices", "last_page_len", "loc")}
    with pytest.raises(ValueError, match="num_qo_heads"):
        group.DecodeGroup([{"kind": "a", "w": {}}], 1, 64, "cpu", attn=attn)


def test_group_layers_of_a_kind_share_shapes():
    w1 = {"w_gate": torch.zeros(32, 64)}
    w2 = {"w_gate": torch.zeros(64, 64)}
    with pytest.raises(ValueError, match="share"):
        group.DecodeGroup([{"kind": "g", "w": w1}, {"kind": "g", "w": w2}], 1, 64, "cpu")
