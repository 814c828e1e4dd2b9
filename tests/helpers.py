"""Comparison helpers shared by the GPU tests."""

import torch

D = 128


def near_exact(got, ref, frac=0.999):
    """Nearly all values equal; the rest within one bf16 ulp of their head
    row's largest value (a flipped rounding of a normalised channel moves
    the RoPE sum by an ulp of its larger term)."""
    got, ref = got.float(), ref.float()
    assert torch.isfinite(got).all()
    head_max = ref.reshape(*ref.shape[:-1], -1, D).abs().amax(-1, keepdim=True)
    bound = (head_max * 2.0 ** -7).expand(*ref.shape[:-1], -1, D).reshape(ref.shape)
    bad = ((got - ref).abs() > bound).nonzero()
    assert bad.shape[0] == 0, (f"{bad.shape[0]} values off by more than an ulp, first {bad[:4].tolist()}, "
                               f"max diff {(got - ref).abs().max().item()}")
    assert (got == ref).float().mean().item() >= frac
