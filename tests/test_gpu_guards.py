"""Guards of the C ABI against arguments the host cannot fully check.

* fa_decode_fwd refuses a split plan whose num_splits * split_span misses
  visible keys (they would be dropped silently) before it launches anything.
* rotary_kernel reads cos/sin rows at positions taken from device-resident
  lengths; a position outside the table rotates to NaN instead of reading past
  the table (the reference's `rotate`, flash_attn_mps/kernels/cache.metal:58-76,
  has no such bound).
"""
import pytest
import torch

from flash_attn_mps_amd import _lib
from flash_attn_mps_amd._cache import rotary
from harness import kernel_args

pytestmark = pytest.mark.gpu


def _decode_args(device, keys, keep):
    q = torch.randn(1, 4, 64, device=device, dtype=torch.bfloat16)
    k = torch.randn(keys, 2, 64, device=device, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    out = torch.empty(1, 4, 64, device=device, dtype=torch.bfloat16)
    lse = torch.empty(4, 1, device=device, dtype=torch.float32)
    cu_q = torch.tensor([0, 1], device=device, dtype=torch.int32)
    cu_k = torch.tensor([0, keys], device=device, dtype=torch.int32)
    keep += [q, k, v, out, lse, cu_q, cu_k]
    return kernel_args(q, k, v, out, lse, keep=keep, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=1,
                       max_seqlen_k=keys)


def test_decode_rejects_a_split_plan_that_drops_keys(device):
    keep = []
    a = _decode_args(device, 300, keep)
    a.num_splits, a.split_span = 1, 128
    with pytest.raises(RuntimeError, match="does not cover"):
        _lib.call("fa_decode_fwd", a, device)
    # A left window shrinks what must be covered: 128 keys of a 127-key window.
    a.window_left = 127
    _lib.call("fa_decode_fwd", a, device)
    torch.cuda.synchronize()


@pytest.mark.parametrize("interleaved", [True, False])
def test_rotary_positions_outside_the_table_become_nan(device, interleaved):
    rows, half = 8, 16
    q = torch.randn(2, 3, 2, 64, device=device, dtype=torch.float16)
    k = torch.randn(2, 3, 1, 64, device=device, dtype=torch.float16)
    cos = torch.rand(rows, half, device=device)
    sin = torch.rand(rows, half, device=device)
    lengths = torch.tensor([4, 6], device=device, dtype=torch.int32)   # K of request 1: 6, 7, 8
    _, k_rot = rotary(q, k, cos, sin, lengths, rotary_interleaved=interleaved)
    torch.cuda.synchronize()
    rot = k_rot[..., : 2 * half].float().cpu()
    assert torch.isfinite(rot[0]).all() and torch.isfinite(rot[1, :2]).all()
    assert torch.isnan(rot[1, 2]).all()
    # Dims past the rotary part are copied whatever the position.
    assert torch.equal(k_rot[..., 2 * half:].cpu(), k[..., 2 * half:].cpu())
