"""FP8 block-scaled dequant and MX upcast kernels (HIP) against the oracle, bit for bit
(NaN where the oracle has NaN): every e4m3 code, every e2m1 nibble, scale bytes 0 and 0xFF,
ragged rows, every output dtype, the axis handling of the reference."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from vaayu_amd import block_formats as bf

pytestmark = pytest.mark.gpu
OUTS = [torch.bfloat16, torch.float16, torch.float32]
ACT = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}


def _eq(a, b):
    return np.array_equal(np.asarray(a, np.float32), np.asarray(b, np.float32), equal_nan=True)


def _e8m0(u8):
    u = np.asarray(u8, np.uint8)
    return np.where(u == 255, np.float32(np.nan), (u.astype(np.uint32) << 23).view(np.float32))


@pytest.mark.parametrize("out", OUTS, ids=["bf16", "fp16", "fp32"])
def test_every_e4m3_code(out):
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8).repeat(64, 1)      # [64, 256]
    scale = torch.tensor([[0.75, 3.0]], dtype=torch.float32).repeat(1, 1)           # bo 64, bi 128
    got = bf.dequantize_block_scaled(codes.cuda().view(torch.float8_e4m3fn), scale.cuda(), out)
    want = O.dequant_block_scaled(codes.numpy(), scale.numpy(), ACT[out])
    assert _eq(got.float().cpu().numpy(), want)


@pytest.mark.parametrize("shape,grid", [((768, 2048), (6, 16)), ((2048, 768), (16, 6)),
                                        ((384, 256), (3, 2)), ((200, 64), (200, 4)),
                                        ((7168, 2048), (56, 16))],
                         ids=["qwen3-gate", "qwen3-down", "blocks", "per-row-bi16", "dsv3-gate"])
@pytest.mark.parametrize("sdt", [torch.float32, torch.bfloat16, torch.float16, "e8m0"])
def test_block_scaled_matches_the_oracle(shape, grid, sdt):
    g = torch.Generator().manual_seed(hash((shape, str(sdt))) % 1000)
    w = torch.randint(0, 256, shape, generator=g, dtype=torch.int32).to(torch.uint8)
    if sdt == "e8m0":
        sc = torch.randint(100, 150, grid, generator=g, dtype=torch.int32).to(torch.uint8)
        sc[0, 0], sc[-1, -1] = 0, 255
        s_np, dev_sc = _e8m0(sc.numpy()), sc.cuda()
    else:
        sc = (torch.rand(grid, generator=g) * 4 + 1e-3).to(sdt)
        s_np, dev_sc = sc.float().numpy(), sc.cuda()
    got = bf.dequantize_block_scaled(w.cuda().view(torch.float8_e4m3fn), dev_sc, torch.bfloat16)
    assert _eq(got.float().cpu().numpy(), O.dequant_block_scaled(w.numpy(), s_np, "bf16"))


def test_the_reference_block_scaled_test_on_the_gpu():
    """tests/test_deepseek_v4_linear.py:306-323 (two geometries), on the kernel."""
    for shape, block in (((256, 512), (128, 128)), ((64, 128), (32, 64))):
        torch.manual_seed(0)
        weight = torch.randn(*shape).to(torch.float8_e4m3fn)
        scale = torch.randn(shape[0] // block[0], shape[1] // block[1]).exp().to(torch.float8_e8m0fnu)
        got = bf.dequantize_block_scaled(weight.cuda(), scale.cuda())
        expanded = scale.float().repeat_interleave(block[0], 0).repeat_interleave(block[1], 1)
        assert torch.equal(got.cpu(), (weight.float() * expanded).bfloat16())


@pytest.mark.parametrize("out", OUTS, ids=["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("k", [2048, 768, 96, 48, 30, 2])
def test_mxfp4_matches_the_oracle(out, k):
    g = torch.Generator().manual_seed(k)
    rows = 37
    q = torch.randint(0, 256, (rows, k // 2), generator=g, dtype=torch.int32).to(torch.uint8)
    s = torch.randint(110, 140, (rows, (k + 31) // 32), generator=g, dtype=torch.int32).to(torch.uint8)
    s[0, 0], s[1, -1], s[2, 0], s[3, 0] = 255, 0, 254, 1
    got = bf.upcast_from_mxfp(q.cuda(), s.cuda(), out, axis=-1)
    assert _eq(got.float().cpu().numpy(), O.upcast_mxfp4(q.numpy(), s.numpy(), ACT[out]))


def test_every_e2m1_pair_and_scale():
    q = torch.arange(256, dtype=torch.int32).to(torch.uint8).reshape(16, 16)    # all pairs
    s = torch.arange(0, 256, 16, dtype=torch.int32).to(torch.uint8).reshape(16, 1)
    s[-1, 0] = 255
    got = bf.upcast_from_mxfp(q.cuda(), s.cuda(), torch.float32, axis=1)
    assert _eq(got.cpu().numpy(), O.upcast_mxfp4(q.numpy(), s.numpy(), "fp32"))


@pytest.mark.parametrize("k", [2048, 64, 40])
def test_mx_e4m3_matches_the_oracle(k):
    g = torch.Generator().manual_seed(k + 1)
    q = torch.randint(0, 256, (19, k), generator=g, dtype=torch.int32).to(torch.uint8)
    s = torch.randint(115, 135, (19, (k + 31) // 32), generator=g, dtype=torch.int32).to(torch.uint8)
    s[0, 0] = 255
    got = bf.upcast_from_mxfp(q.cuda().view(torch.float8_e4m3fn), s.cuda(), torch.bfloat16, axis=1)
    assert _eq(got.float().cpu().numpy(), O.upcast_mx_e4m3(q.numpy(), s.numpy(), "bf16"))


def test_mx_along_a_leading_axis_of_a_3d_tensor():
    g = torch.Generator().manual_seed(4)
    q = torch.randint(0, 256, (3, 32, 5), generator=g, dtype=torch.int32).to(torch.uint8)  # axis 1
    s = torch.randint(120, 130, (3, 2, 5), generator=g, dtype=torch.int32).to(torch.uint8)
    got = bf.upcast_from_mxfp(q.cuda(), s.cuda(), torch.bfloat16, axis=1)
    cpu = bf.upcast_from_mxfp(q, s, torch.bfloat16, axis=1)
    assert got.shape == (3, 64, 5) and torch.equal(got.cpu(), cpu)
