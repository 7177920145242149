"""The restated acceptance bar (tests/fidelity.py) on the CPU: identical pages
score 1, the score is the cosine of attention outputs (GQA) or weights (MLA)
computed in closed form for a page of one token, and it falls as the decoded
page drifts."""
import math

import torch

from fidelity import attention_fidelity, reference_pages


def test_identical_pages_score_one():
    k, v = reference_pages(16, 8, 128, 64, False, 1, torch.float32)
    assert abs(attention_fidelity(k[0], v[0], k[0], v[0]) - 1.0) < 1e-6
    k, _ = reference_pages(64, 1, 576, 64, True, 1, torch.float32)
    assert abs(attention_fidelity(k[0], None, k[0], None) - 1.0) < 1e-6


def test_one_token_page_reduces_to_the_value_cosine():
    """With one token the softmax weight is 1 for both pages, so the GQA score
    is the cosine of the V rows (over all heads) whatever K holds."""
    g = torch.Generator().manual_seed(5)
    k = torch.randn((1, 4, 32), generator=g)
    v = torch.randn((1, 4, 32), generator=g)
    vh = v + 0.3 * torch.randn((1, 4, 32), generator=g)
    want = float((v * vh).sum() / (v.norm() * vh.norm()))
    assert math.isclose(attention_fidelity(k, v, k * 3.0, vh), want, rel_tol=1e-6)


def test_score_falls_with_the_error():
    k, v = reference_pages(16, 8, 128, 64, False, 1, torch.float32)
    g = torch.Generator().manual_seed(1)
    noise = torch.randn(k[0].shape, generator=g)
    s = [attention_fidelity(k[0], v[0], k[0] + e * noise, v[0] + e * noise) for e in (0.01, 0.05, 0.2)]
    assert 1.0 > s[0] > s[1] > s[2]


def test_reference_pages_follow_the_reference_generator():
    """The RoPE columns carry linspace(-4.5, 4.5) * sin(t): at t = 0 they are
    N(0, 0.4) only; V is N(0, 0.25)."""
    k, v = reference_pages(64, 8, 128, 64, False, 4, torch.float32)
    assert abs(k[:, 0, :, :64].std().item() - 0.4) < 0.05
    assert k[:, 1:, :, 0].abs().mean() > 1.0 and abs(v.std().item() - 0.25) < 0.01
