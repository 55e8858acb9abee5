"""Writes the golden fixtures of tests/golden/ (run from the repo root:
``python tests/golden/make_golden.py``).

Every expected value comes from torch's own CPU arithmetic, never from the
oracle under test and never from the reference's code:

* e4m3.npz -- the E4M3FN decode table of all 256 codes (torch's
  float8_e4m3fn -> float32 cast) and the encode known-answer table of
  flash_attn_mps tests/test_cache.py:39-54 (127 finite codes, the 126
  midpoints between them, both signs, +-1000 and +-inf), expected codes
  = clamp(x, -448, 448) cast to float8_e4m3fn, as that test computes them;
* merge.npz -- the extreme-LSE pair-merge table of flash_attn_mps
  tests/test_merge.py:14-15 with expected LSE = torch.logaddexp and
  expected outputs from the weights exp(lse_side - lse) of that test;
* sdpa.npz -- one varlen GQA causal case (fp64) with expected outputs
  from torch.nn.functional.scaled_dot_product_attention per request.
"""
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent


def e4m3():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    decoded = codes.view(torch.float8_e4m3fn).float()
    representable = torch.arange(127, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float()
    ties = (representable[:-1] + representable[1:]) / 2
    values = torch.cat((representable, ties, -representable, -ties,
                        torch.tensor([1000.0, -1000.0, float("inf"), -float("inf")])))
    expected = values.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    np.savez(HERE / "e4m3.npz", decode_codes=codes.numpy(), decode_values=decoded.numpy(),
             encode_inputs=values.numpy(), encode_codes=expected.numpy())


def merge():
    g = torch.Generator().manual_seed(11)
    la = torch.tensor([[1000., -1000., -float("inf")], [-float("inf"), 0., 10.], [-float("inf"), -50., 50.]],
                      dtype=torch.float64)
    lb = torch.tensor([[1001., -1001., 0.], [-float("inf"), -float("inf"), 11.], [1., 50., -50.]],
                      dtype=torch.float64)
    left = torch.randn(3, 3, 7, generator=g, dtype=torch.float64)
    right = torch.randn(3, 3, 7, generator=g, dtype=torch.float64)
    le = torch.logaddexp(la, lb)
    wa = (la - le).exp().nan_to_num(0).T.unsqueeze(-1)
    wb = (lb - le).exp().nan_to_num(0).T.unsqueeze(-1)
    out = wa * left + wb * right
    np.savez(HERE / "merge.npz", left=left.numpy(), right=right.numpy(), left_lse=la.numpy(),
             right_lse=lb.numpy(), out=out.numpy(), lse=le.numpy())


def sdpa():
    g = torch.Generator().manual_seed(12)
    q_lens, k_lens, hq, hkv, d = [3, 6], [7, 6], 4, 2, 16
    q = torch.randn(sum(q_lens), hq, d, generator=g, dtype=torch.float64)
    k = torch.randn(sum(k_lens), hkv, d, generator=g, dtype=torch.float64)
    v = torch.randn(sum(k_lens), hkv, d, generator=g, dtype=torch.float64)
    outs, qs, ks = [], 0, 0
    for n, m in zip(q_lens, k_lens):
        mask = torch.ones(n, m, dtype=torch.bool).tril(m - n)
        o = F.scaled_dot_product_attention(q[qs:qs + n].transpose(0, 1),
                                           k[ks:ks + m].repeat_interleave(2, 1).transpose(0, 1),
                                           v[ks:ks + m].repeat_interleave(2, 1).transpose(0, 1),
                                           attn_mask=mask, scale=0.25)
        outs.append(o.transpose(0, 1))
        qs, ks = qs + n, ks + m
    np.savez(HERE / "sdpa.npz", q=q.numpy(), k=k.numpy(), v=v.numpy(), q_lens=np.array(q_lens),
             k_lens=np.array(k_lens), scale=np.array(0.25), out=torch.cat(outs).numpy())


if __name__ == "__main__":
    e4m3()
    merge()
    sdpa()
