"""The FP8 block-scaled and MX mirrors on CPU tensors (the reference's eager arithmetic)
against the oracle, and their argument checks. The HIP kernels are held to the same oracle
in test_gpu_block_formats.py."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from vaayu_amd import block_formats as bf


def _eq(a, b):
    return np.array_equal(np.asarray(a, np.float32), np.asarray(b, np.float32), equal_nan=True)


@pytest.mark.parametrize("shape,grid", [((256, 512), (2, 4)), ((96, 64), (96, 4)), ((48, 32), (3, 2))])
@pytest.mark.parametrize("sdt", [torch.float32, torch.bfloat16, "e8m0"])
def test_block_scaled_cpu_matches_the_oracle(shape, grid, sdt):
    g = torch.Generator().manual_seed(1)
    w = torch.randint(0, 256, shape, generator=g, dtype=torch.int32).to(torch.uint8)
    if sdt == "e8m0":
        sc = torch.randint(110, 140, grid, generator=g, dtype=torch.int32).to(torch.uint8)
        s_np = np.where(sc.numpy() == 255, np.nan, (sc.numpy().astype(np.uint32) << 23).view(np.float32))
    else:
        sc = (torch.rand(grid, generator=g) + 0.01).to(sdt)
        s_np = sc.float().numpy()
    got = bf.dequantize_block_scaled(w.view(torch.float8_e4m3fn), sc, torch.bfloat16)
    want = O.dequant_block_scaled(w.numpy(), s_np, "bf16")
    assert _eq(got.float().numpy(), want)


@pytest.mark.parametrize("k", [64, 48, 30])
def test_mxfp4_cpu_matches_the_oracle(k):
    g = torch.Generator().manual_seed(2)
    q = torch.randint(0, 256, (5, k // 2), generator=g, dtype=torch.int32).to(torch.uint8)
    s = torch.randint(100, 150, (5, (k + 31) // 32), generator=g, dtype=torch.int32).to(torch.uint8)
    s[0, 0], s[1, -1] = 255, 0
    got = bf.upcast_from_mxfp(q, s, torch.bfloat16, axis=-1)
    assert _eq(got.float().numpy(), O.upcast_mxfp4(q.numpy(), s.numpy(), "bf16"))


def test_mx_axis_follows_the_reference_layout():
    g = torch.Generator().manual_seed(3)
    q = torch.randint(0, 256, (16, 6), generator=g, dtype=torch.int32).to(torch.uint8)   # axis 0
    s = torch.randint(120, 130, (1, 6), generator=g, dtype=torch.int32).to(torch.uint8)
    got = bf.upcast_from_mxfp(q.T.contiguous().T, s, torch.float32, axis=0)
    want = O.upcast_mxfp4(q.T.numpy(), s.T.numpy(), "fp32").T
    assert got.shape == (32, 6) and _eq(got.numpy(), want)


def test_bad_arguments_raise():
    with pytest.raises(ValueError):
        bf.dequantize_block_scaled(torch.zeros(10, 16, dtype=torch.float8_e4m3fn), torch.ones(3, 1))
    with pytest.raises(TypeError):
        bf.upcast_from_mxfp(torch.zeros(2, 16), torch.zeros(2, 1, dtype=torch.uint8), torch.bfloat16, -1)
    with pytest.raises(ValueError):
        bf.upcast_from_mxfp(torch.zeros(2, 16, dtype=torch.uint8), torch.zeros(2, 3, dtype=torch.uint8),
                            torch.bfloat16, -1)
