"""Selection quality on planted retrieval structure (the reference's
tests/test_selection.py:43-65 with the structured fixture of
tests/conftest.py:36-39): every HIP selector must recover at least the
fraction of attention mass that its fraction of kept blocks would give, and
the Quest GQA union must read at least as much as per-head lists."""

from __future__ import annotations

import pytest
import torch

from linattn_amd.kernels.prefill import block_select_hip
from linattn_amd.kernels.quest_pages import page_update_hip, quest_select_hip
from linattn_amd.kernels.routing import gate_select_hip, xattn_select_hip
from linattn_amd.core import AttnConfig
from linattn_amd.registry import build
from structured import block_recall, lists_to_mask, structured_inputs

pytestmark = pytest.mark.gpu

# the reference's test configuration (tests/conftest.py:13-27)
CFG = dict(n_heads=4, n_kv_heads=2, head_dim=32, block_size=16, window_size=32,
           topk_blocks=3, topk_tokens=48, compress_ratio=8, sink_size=2, stride=4)
T = 192


@pytest.fixture(scope="module")
def structured():
    return structured_inputs(1, CFG["n_heads"], T, CFG["head_dim"], kv_heads=CFG["n_kv_heads"],
                             seed=1)


def selector_mask(name, q, k, dev):
    bs = CFG["block_size"]
    qd, kd = q.to(dev), k.to(dev)
    if name == "quest":
        mn, mx = page_update_hip(kd, bs)
        ids, _ = quest_select_hip(qd, mn, mx, page_size=bs, topk=CFG["topk_blocks"], offset=0,
                                  gqa_union=False)
        return lists_to_mask(ids, bs, T)
    if name == "minference":  # the block-sparse estimator of _block_sparse
        ids, _ = block_select_hip(qd, kd, block=bs, topk=CFG["topk_blocks"], sink_blocks=1,
                                  window_blocks=1)
        return lists_to_mask(ids, bs, T, rows_per_block=bs)
    if name == "moba":
        ids, _ = gate_select_hip(qd, kd, block=bs, topk=CFG["topk_blocks"], offset=0)
        return lists_to_mask(ids, bs, T)
    if name == "xattention":
        ids, _ = xattn_select_hip(qd, kd, block=8, stride=CFG["stride"], threshold=0.9)
        return lists_to_mask(ids, 8, T, rows_per_block=8)
    if name == "dsa":
        var = build("hip_dsa", AttnConfig(**CFG))
        ids = var.select_lists(qd, kd, 0)
        return lists_to_mask(ids, 1, T)
    raise KeyError(name)


@pytest.mark.parametrize("name", ["quest", "minference", "moba", "xattention", "dsa"])
def test_selection_recovers_mass_on_structured_inputs(dev, structured, name):
    q, k, _ = structured
    mask = selector_mask(name, q, k, dev)
    assert bool(mask.any(-1).all()), f"{name} left a query with nothing to read"
    recall, budget = block_recall(mask, q, k, CFG["block_size"])
    assert recall >= budget, f"{name} recall {recall:.3f} below its budget {budget:.3f}"


def test_quest_gqa_union_inflates_budget(dev, structured):
    """The union over a GQA group reads at least as many keys as per-head lists."""
    q, k, _ = structured
    bs = CFG["block_size"]
    mn, mx = page_update_hip(k.to(dev), bs)
    reads = {}
    for union in (True, False):
        ids, _ = quest_select_hip(q.to(dev), mn, mx, page_size=bs, topk=CFG["topk_blocks"],
                                  offset=0, gqa_union=union)
        m = lists_to_mask(ids, bs, T)
        if union:  # (B, Hkv, T, T) lists serve every query head of the group
            m = m.repeat_interleave(CFG["n_heads"] // CFG["n_kv_heads"], dim=1)
        reads[union] = float(m.sum(-1).float().mean())
    assert reads[True] >= reads[False] > 0
