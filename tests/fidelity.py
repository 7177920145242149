"""The reference's acceptance bar for decoded pages, restated for the tests.

research/benchmarks/bench_cold_page_pipeline.py:97-146 scores a decoded page
by simulated single-page attention: a query q ~ N(0, 1) (seed 99) of one
head-dim vector per KV head attends over the page's tokens,
logits[h, t] = q[h] . k[t, h] / sqrt(head_dim), softmax over t.  With V (GQA)
the score is the cosine between the attention outputs sum_t a[h, t] v[t, h]
of the original and the decoded page; without V (single-buffer MLA) it is the
cosine between the attention weights.  The reference asserts a score above
0.995 (bench_cold_page_pipeline.py:313, :965-971).

reference_pages restates the reference's page generator
(bench_cold_page_pipeline.py:69-93), the data that bar is asserted on: K ~
N(0, 0.4) with linspace(-4.5, 4.5, rope_dim) * sin(token) added to the RoPE
columns, V ~ N(0, 0.25).
"""
from __future__ import annotations

import torch

BAR = 0.995


def attention_fidelity(k_ref: torch.Tensor, v_ref: torch.Tensor | None, k_hat: torch.Tensor,
                       v_hat: torch.Tensor | None, seed: int = 99) -> float:
    """Score of one page [T, H, D] (float32 on the CPU)."""
    kr, kh = k_ref.detach().float().cpu(), k_hat.detach().float().cpu()
    T, H, D = kr.shape
    q = torch.randn((H, 1, D), generator=torch.Generator().manual_seed(seed))
    scale = D ** -0.5
    # [H, 1, D] x [H, D, T] -> [H, 1, T]
    lr = torch.matmul(q, kr.permute(1, 2, 0).contiguous()) * scale
    lh = torch.matmul(q, kh.permute(1, 2, 0).contiguous()) * scale
    ar, ah = torch.softmax(lr, dim=-1), torch.softmax(lh, dim=-1)
    if v_ref is None:
        return torch.nn.functional.cosine_similarity(ar.reshape(-1), ah.reshape(-1), dim=0).item()
    vr, vh = v_ref.detach().float().cpu(), v_hat.detach().float().cpu()
    # [H, 1, T] x [H, T, D] -> [H, 1, D]
    outr = torch.matmul(ar, vr.permute(1, 0, 2).contiguous())
    outh = torch.matmul(ah, vh.permute(1, 0, 2).contiguous())
    return torch.nn.functional.cosine_similarity(outr.reshape(-1), outh.reshape(-1), dim=0).item()


def reference_pages(num_tokens: int, num_heads: int, head_dim: int, rope_dim: int, mla: bool, n: int,
                    dtype: torch.dtype, seed: int = 42):
    """n pages [n, T, H, D] of the reference benchmark's distribution (CPU)."""
    g = torch.Generator().manual_seed(seed)
    shape = (n, num_tokens, num_heads, head_dim)
    k = torch.randn(shape, generator=g) * 0.4
    if rope_dim > 0:
        ramp = torch.linspace(-4.5, 4.5, rope_dim).reshape(1, 1, 1, rope_dim)
        k[..., :rope_dim] += ramp * torch.sin(torch.arange(num_tokens, dtype=torch.float32)).reshape(1, -1, 1, 1)
    v = None if mla else torch.randn(shape, generator=g) * 0.25
    return k.to(dtype), (None if v is None else v.to(dtype))
