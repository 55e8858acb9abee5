"""Host-side contract of the public API, checked without a GPU: training
features are refused with NotImplementedError and host tensors with
ValueError before anything is launched (the behaviour pinned by flash_attn_mps
tests/test_interface.py:190-195), and the vLLM-only options refuse the same
way (flash_attn_mps/vllm.py:48-57)."""
import pytest
import torch

import flash_attn_mps_amd as fa
from flash_attn_mps_amd import vllm
from flash_attn_mps_amd._problem import MaskSpec, Want


def _dense():
    return torch.randn(1, 2, 2, 16)


@pytest.mark.parametrize("kwargs,match", [
    (dict(dropout_p=0.1), "dropout"),
    (dict(return_attn_probs=True), "return_softmax_lse"),
])
def test_training_options_are_refused(kwargs, match):
    q = _dense()
    with pytest.raises(NotImplementedError, match=match):
        fa.flash_attn_func(q, q, q, **kwargs)


def test_autograd_inputs_are_refused():
    q = _dense().requires_grad_()
    with pytest.raises(NotImplementedError, match="grad"):
        fa.flash_attn_func(q, q.detach(), q.detach())


def test_host_tensors_are_refused():
    q = _dense()
    with pytest.raises(ValueError, match="GPU"):
        fa.flash_attn_func(q, q, q)
    cu = torch.tensor([0, 2], dtype=torch.int32)
    with pytest.raises(ValueError, match="GPU"):
        fa.flash_attn_varlen_func(q[0], q[0], q[0], cu, cu, 2, 2)
    with pytest.raises(ValueError, match="GPU"):
        fa.store_kvcache(q[0], q[0], q, q, cu[:2])


@pytest.mark.parametrize("option", [
    dict(q_v=torch.zeros(1)), dict(cp_world_size=2), dict(cp_rank=1), dict(cp_tot_seqused_k=torch.zeros(1)),
    dict(block_sparse_tensors=object()), dict(output_scale=torch.ones(1)), dict(aux_tensor_leading_dims=(1,)),
])
def test_vllm_options_outside_the_contract(option):
    q = _dense()[0]
    cu = torch.tensor([0, 2], dtype=torch.int32)
    with pytest.raises(NotImplementedError):
        vllm.flash_attn_varlen_func(q, q, q, 2, cu, 2, cu_seqlens_k=cu, **option)


def test_vllm_version_hint_and_mask_descriptors():
    q = _dense()[0]
    cu = torch.tensor([0, 2], dtype=torch.int32)
    with pytest.raises(ValueError, match="fa_version"):
        vllm.flash_attn_varlen_func(q, q, q, 2, cu, 2, cu_seqlens_k=cu, fa_version=1)
    assert vllm.mm_prefix_mask() == MaskSpec(1, -1, False)
    assert vllm.mm_prefix_mask(16, True) == MaskSpec(1, 16, True)
    assert vllm.rswa_mask() == MaskSpec(2)
    for bad in (0, -2):
        with pytest.raises(ValueError):
            vllm.mm_prefix_mask(bad)
    with pytest.raises(ValueError):
        vllm.mm_prefix_mask(None, True)
    assert vllm.get_scheduler_metadata(1, 2, x=3) is None


def test_want_reports_shape_dtype_and_device():
    t = torch.zeros(3, 4, dtype=torch.int64)
    Want("x", (3, None), (torch.int64,)).check(t, t.device)
    Want("x", {(4,), (3, 4)}).check(t, t.device)
    with pytest.raises(ValueError, match=r"\[3, 5\]"):
        Want("x", (3, 5)).check(t, t.device)
    with pytest.raises(TypeError, match="int32"):
        Want("x", None, (torch.int32,), TypeError).check(t, t.device)
    with pytest.raises(ValueError, match="device"):
        Want("x").check(t, torch.device("meta"))
