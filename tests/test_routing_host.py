"""Host-side arguments of the router's Python layer (no GPU): the
MOE_APPROX_TOPK switches and the recall target's range."""
import pytest
import torch

from dw_tpu_amd import routing


def test_env_flag(monkeypatch):
    for v, want in (("1", True), ("true", True), ("ON", True), ("0", False), ("", False), ("no", False)):
        monkeypatch.setenv("MOE_APPROX_TOPK", v)
        assert routing._env_flag("MOE_APPROX_TOPK") is want
    monkeypatch.delenv("MOE_APPROX_TOPK")
    assert routing._env_flag("MOE_APPROX_TOPK") is False


@pytest.mark.parametrize("target", [0.0, -0.5, 1.5])
def test_recall_target_range(target):
    with pytest.raises(ValueError, match="recall_target"):
        routing.fused_moe_fp4_routing(torch.zeros(4, 8), 2, False, "softmax", torch.float32, {}, approx_topk=True,
                                      recall_target=target)


def test_recall_target_from_env(monkeypatch):
    monkeypatch.setenv("MOE_APPROX_TOPK_RECALL_TARGET", "2")
    with pytest.raises(ValueError, match="recall_target"):
        routing.fused_moe_fp4_routing(torch.zeros(4, 8), 2, False, "softmax", torch.float32, {}, approx_topk=True)


def test_host_tensor_still_rejected():
    with pytest.raises(ValueError, match="device tensor"):
        routing.fused_moe_fp4_routing(torch.zeros(4, 8), 2, False, "softmax", torch.float32, {}, approx_topk=True)


@pytest.mark.parametrize("value", ["2", "not-a-number"])
def test_recall_target_env_ignored_off_the_approx_branch(monkeypatch, value):
    """The recall target is read only when the approx_max_k branch is taken:
    with approx off (or hash routing given) a malformed value is ignored and
    the call proceeds to its usual checks (here: host tensors are rejected)."""
    monkeypatch.setenv("MOE_APPROX_TOPK_RECALL_TARGET", value)
    monkeypatch.delenv("MOE_APPROX_TOPK", raising=False)
    with pytest.raises(ValueError, match="device tensor"):
        routing.fused_moe_fp4_routing(torch.zeros(4, 8), 2, False, "softmax", torch.float32, {})
    with pytest.raises(ValueError, match="device tensor"):
        routing.fused_moe_fp4_routing(torch.zeros(4, 8), 2, False, "softmax", torch.float32,
                                      {"hash_based_topk_indices": torch.zeros(4, 2, dtype=torch.int32)},
                                      approx_topk=True)
