"""GPU tests of the head layout kernels (csrc/layout.hip): bit-exact against
torch's permutes, both directions, through autograd, on the vector path and the
element path (head dims that are not a multiple of the 16-byte vector)."""

import pytest
import torch

from ferrite.kernels.heads import merge_heads, split_heads

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("b,s,g,h,d,dtype", [
    (8, 1024, 3, 12, 64, torch.bfloat16),   # the GPT's qkv
    (2, 77, 1, 5, 24, torch.float32),
    (1, 9, 3, 2, 7, torch.bfloat16),        # element path
    (3, 5, 4, 1, 128, torch.float32),
])
def test_split_merge_exact(dev, b, s, g, h, d, dtype):
    x = torch.randn(b, s, g * h * d, device=dev).to(dtype)
    parts = split_heads(x, g, h)
    want = x.reshape(b, s, g, h, d).permute(2, 0, 3, 1, 4)
    assert len(parts) == g
    for i, p in enumerate(parts):
        assert p.is_contiguous() and p.shape == (b, h, s, d)
        assert torch.equal(p, want[i])
    back = merge_heads(*parts)
    assert torch.equal(back, x)


def test_autograd_round_trip(dev):
    x = torch.randn(2, 16, 3 * 4 * 8, device=dev, dtype=torch.bfloat16, requires_grad=True)
    q, k, v = split_heads(x, 3, 4)
    o = merge_heads(q * 2 + k)  # [2, 16, 32]
    cot = torch.randn_like(o)
    (o * cot).sum().backward()
    c = cot.reshape(2, 16, 4, 8)
    want = torch.cat([(2 * c), c, torch.zeros_like(c)], dim=2).reshape(2, 16, 96)
    assert torch.equal(x.grad, want.to(x.grad.dtype))


def test_validation(dev):
    with pytest.raises(ValueError):
        split_heads(torch.zeros(2, 3, 10, device=dev), 3, 2)
    with pytest.raises(ValueError):
        merge_heads(torch.zeros(1, 2, 3, 4, device=dev), torch.zeros(1, 2, 3, 5, device=dev))
