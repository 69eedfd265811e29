"""Synthetic packed experts on any device: the repo's symmetric group quantizer in torch.

The quantizer is the one Vaayu's tests pack checkpoints with
(tests/test_packed_expert_dequant.py:44-57): per group of `group_size` along a row,
scale = max|w| (clamped to 1e-6) / (2^(bits-1) - 1) in fp32, codes = round-half-even(w /
scale) clamped to the signed range, packed compressed-tensors style (offset 2^(bits-1), a
row a little-endian bit stream, 32/bits codes per int32 word). Used to build
benchmark-sized expert sets directly in HBM.
"""
import torch

from .moe_patch import build_expert_blob

ROLE_SHAPES = ("gate", "down", "up")


def quantize_pack(weight: torch.Tensor, num_bits: int, group_size: int,
                  scale_dtype=torch.float16):
    """(packed int32 [rows, cols*bits/32], scale [rows, cols/group]) of `weight`."""
    if 32 % num_bits:
        raise ValueError("packing here needs a bit width dividing 32")
    rows, cols = weight.shape
    g = weight.float().reshape(rows, cols // group_size, group_size)
    qmax = 2 ** (num_bits - 1) - 1
    scale = g.abs().amax(dim=-1).clamp(min=1e-6) / qmax
    q = torch.round(g / scale.unsqueeze(-1)).clamp(-qmax - 1, qmax).to(torch.int32)
    u = (q.reshape(rows, cols) + (1 << (num_bits - 1))).reshape(rows, -1, 32 // num_bits)
    shifts = torch.arange(32 // num_bits, device=weight.device, dtype=torch.int64) * num_bits
    words = (u.to(torch.int64) << shifts).sum(dim=-1)
    words = torch.where(words >= 2 ** 31, words - 2 ** 32, words).to(torch.int32)
    return words, scale.to(scale_dtype)


def random_expert(hidden: int, inter: int, num_bits: int, group_size: int, *, generator,
                  device, std: float = 0.02, scale_dtype=torch.float16) -> dict:
    """One expert: bf16 N(0, std) gate/down/up weights, quantized and built into a blob."""
    by_role = {}
    for role, shape in (("gate", (inter, hidden)), ("down", (hidden, inter)),
                        ("up", (inter, hidden))):
        w = (torch.randn(shape, generator=generator, device=device) * std).to(torch.bfloat16)
        packed, scale = quantize_pack(w, num_bits, group_size, scale_dtype)
        by_role[role] = {"weight_packed": packed, "weight_scale": scale,
                         "weight_shape": torch.tensor(list(shape))}
    return build_expert_blob(by_role)


def clone_blob(blob: dict) -> dict:
    """Same bytes at new addresses (a distinct copy in HBM)."""
    return {"flat": {n: t.clone() for n, t in blob["flat"].items()}, "geom": blob["geom"]}
