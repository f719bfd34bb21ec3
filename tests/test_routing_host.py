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
