"""TEST INFRASTRUCTURE ONLY: CPU restatement of the attention-state merges.

merge_pair restates flash_attn_mps/kernels/merge.metal:9-28 (used by
_merge.merge_attn_states, flash_attn_mps/_merge.py:20-41) and merge_partials
merge.metal:30-58 (flash_attn_mps/_merge.py:44-57):

  peak = max_s lse_s;  all -inf -> output 0, LSE -inf;
  w_s = exp(lse_s - peak), except peak = +inf: w_s = [lse_s == +inf];
  out = sum_{w_s > 0} w_s * o_s / sum_s w_s;  lse = peak + log(sum_s w_s).
States with zero weight are never read, so their NaN payloads do not matter.
"""
import torch


def _weights(lse, peak):
    finite_peak = torch.where(torch.isfinite(peak), peak, torch.zeros_like(peak))
    w = torch.exp(lse - finite_peak)
    w = torch.where(peak == torch.inf, (lse == torch.inf).to(lse.dtype), w)
    w = torch.where(peak == -torch.inf, torch.zeros_like(w), w)
    return w


def merge_partials(partial, partial_lse):
    """partial [S, T, H, D], partial_lse [S, H, T] -> (out [T, H, D], lse [H, T]) in float64."""
    o = partial.detach().cpu().double()
    l = partial_lse.detach().cpu().double()
    splits, tokens, heads, dim = o.shape
    peak = l.amax(dim=0) if splits else torch.full((heads, tokens), -torch.inf, dtype=torch.float64)
    w = _weights(l, peak.unsqueeze(0))                              # [S, H, T]
    denom = w.sum(dim=0)                                            # [H, T]
    wt = w.permute(0, 2, 1).unsqueeze(-1)                           # [S, T, H, 1]
    contrib = torch.where(wt > 0, wt * torch.where(wt > 0, o, torch.zeros_like(o)), torch.zeros_like(o))
    num = contrib.sum(dim=0)                                        # [T, H, D]
    empty = (peak == -torch.inf).transpose(0, 1).unsqueeze(-1)     # [T, H, 1]
    out = torch.where(empty, torch.zeros_like(num), num / denom.transpose(0, 1).unsqueeze(-1))
    lse = torch.where(peak == -torch.inf, peak, peak + torch.log(denom))
    return out, lse


def merge_pair(a, a_lse, b, b_lse):
    """a, b [T, H, D]; a_lse, b_lse [H, T] -> (out, lse) in float64."""
    return merge_partials(torch.stack((a.detach().cpu(), b.detach().cpu())),
                          torch.stack((a_lse.detach().cpu(), b_lse.detach().cpu())))
