"""Host-side logic that needs no GPU: the variant registry and contract, the
no-fallback rule, and argument validation of the kernel wrappers."""

from __future__ import annotations

import pytest
import torch

from linattn_amd.core import AttnConfig
from linattn_amd.kernels import backend_for, describe_backends
from linattn_amd.kernels.block_sparse import block_sparse_attention, sparse_attention
from linattn_amd.kernels.fused_indexer import indexer_topk
from linattn_amd.kernels.quest_pages import alloc_page_meta, page_select_hip
from linattn_amd.registry import KERNEL_VARIANTS, build, describe_kernel


def test_registry_names_and_errors():
    """registry.py:225-236: <backend>_<variant> names, KeyError otherwise."""
    assert set(KERNEL_VARIANTS) == {"hip_quest", "hip_dsa", "hip_moba", "hip_xattention",
                                    "hip_sliding_window", "hip_streaming_sink"}
    assert describe_kernel("hip_xattention")["reference"] == "xattention"
    # the three selection rules of selection.py:578-590; anything else is refused
    for mode in ("threshold", "topk", "top_ratio"):
        assert build("hip_xattention", extras={"select_mode": mode}).select_mode == mode
    with pytest.raises(ValueError):
        build("hip_xattention", extras={"select_mode": "top_p"})
    assert describe_kernel("hip_moba")["reference"] == "moba"
    assert describe_kernel("hip_quest")["reference"] == "quest"
    assert build("hip_quest").name == "hip_quest"
    with pytest.raises(KeyError):
        build("hip_nope")
    with pytest.raises(KeyError):
        describe_kernel("quest")


def test_config_contract():
    """core.py:47-78 field names, group size, unknown-field and GQA errors."""
    c = AttnConfig(n_heads=8, n_kv_heads=2)
    assert c.group_size == 4 and c.with_(topk_blocks=9).topk_blocks == 9
    with pytest.raises(TypeError):
        build("hip_quest", AttnConfig(), not_a_field=1)
    with pytest.raises(ValueError):
        build("hip_quest", AttnConfig(n_heads=3, n_kv_heads=2))


def test_cost_model_follows_the_reference_conventions():
    """read_budget / flops / memory_bytes of the torch variants
    (selection.py:118-133, local.py:55-61)."""
    c = AttnConfig(n_heads=4, n_kv_heads=2, head_dim=64, block_size=16, window_size=32,
                   topk_blocks=3, sink_size=2)
    q = build("hip_quest", c)
    assert q.read_budget(1000) == 3 * 16 + 32
    n_pages = (1000 + 15) // 16
    assert q.flops(1000) == 4 * 4 * 1000 * 80 * 64 + 2 * 4 * 1000 * n_pages * 64
    w = build("hip_sliding_window", c)
    assert w.read_budget(1000) == 34 and w.memory_bytes(1000) == 2 * 34 * 64 * 4


def test_cpu_tensors_are_rejected_not_served_on_cpu():
    """There is no CPU fallback (the oracle is not a backend)."""
    q = torch.randn(1, 2, 1, 64)
    k = torch.randn(1, 2, 32, 64)
    ids = torch.zeros(1, 2, 1, 1, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="GPU"):
        sparse_attention(q, k, k, ids, unit=16)
    with pytest.raises(RuntimeError, match="GPU"):
        block_sparse_attention(q, k, k, ids, block_size=16)
    with pytest.raises(RuntimeError, match="GPU"):
        indexer_topk(torch.randn(1, 4, 2, 8), torch.randn(1, 4, 2, 8), torch.rand(1, 4, 2), 2)
    with pytest.raises(RuntimeError, match="GPU"):
        page_select_hip(q, *alloc_page_meta(1, 2, 2, 64, torch.float32, "cpu"), 16, 1)
    with pytest.raises(ValueError):
        block_sparse_attention(q, k, k, ids, block_size=16, backend="triton")


def test_backend_report():
    """kernels/__init__.py:66-95: one backend, 'hip'."""
    assert backend_for() == "hip"
    with pytest.raises(ValueError):
        backend_for("torch")
    info = describe_backends()
    for key in ("platform", "torch", "hip_library", "gpu"):
        assert key in info


def test_page_meta_is_page_minor():
    mn, mx = alloc_page_meta(2, 3, 10, 64, torch.bfloat16, "cpu")
    assert mn.shape == (2, 3, 10, 64) and mn.stride(2) == 1 and mn.stride(3) == 12
