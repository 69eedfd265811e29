"""The whole-blob dequant kernel: bit-exact with the oracle and the eager arithmetic."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import cpu_blobs, to_device
from vaayu_amd import moe_patch as mp

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 128), (8, 64), (2, 64), (1, 128)])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("sdt", [torch.bfloat16, torch.float16, torch.float32])
def test_dequant_is_bit_exact(bits, gs, out_dtype, sdt):
    if bits == 1:       # the repo's quantizer has no 1-bit range (qmax 0): raw codes
        rng = np.random.default_rng(11)
        words = rng.integers(-2 ** 31, 2 ** 31, 4096, dtype=np.int64).astype(np.int32)
        blob = {"flat": {"packed": torch.from_numpy(words),
                         "scale": torch.from_numpy(rng.uniform(1e-3, 1e-1, 4096 * 32 // gs)
                                                   .astype(np.float32)).to(sdt)},
                "geom": (1, gs, ())}
    else:
        (blob,) = cpu_blobs(512, 256, bits, gs, 1, scale_dtype=sdt)
    g = to_device(blob)
    got = mp._hip_dequant(g["flat"]["packed"], g["flat"]["scale"], bits, gs, out_dtype)
    want = O.dequant_flat(blob["flat"]["packed"], blob["flat"]["scale"], bits, gs, out_dtype)
    assert np.array_equal(got.float().cpu().numpy(), want)
    eager = mp._fused_dequant_kernel(g["flat"]["packed"], g["flat"]["scale"], bits, gs, out_dtype)
    assert torch.equal(got, eager)


def test_the_blob_path_uses_the_kernel_and_slices_roles():
    (blob,) = cpu_blobs(2048, 768, 4, 128, 1, scale_dtype=torch.float16)
    g = to_device(blob)
    assert mp._fused_dequant_fn(4, 128, torch.bfloat16, "cuda") is mp._hip_dequant
    dense = mp.dequantize_expert_blob(g, torch.bfloat16)
    wg, wd, wu = O.expert_weights(blob, "bf16")
    for t, o in ((dense["gate"], wg), (dense["down"], wd), (dense["up"], wu)):
        assert np.array_equal(t.float().cpu().numpy(), o)


def test_odd_word_counts_and_tails():
    rng = np.random.default_rng(0)
    for n_words in (1, 3, 5, 257):
        words = torch.from_numpy(rng.integers(-2 ** 31, 2 ** 31, n_words, dtype=np.int64)
                                 .astype(np.int32)).cuda()
        scale = torch.from_numpy(rng.uniform(0.001, 0.1, n_words).astype(np.float32)).half().cuda()
        got = mp._hip_dequant(words, scale, 4, 8, torch.bfloat16)
        want = O.dequant_flat(words.cpu(), scale.cpu(), 4, 8, "bf16")
        assert np.array_equal(got.float().cpu().numpy(), want)


@pytest.mark.parametrize("bits,gs", [(4, 128), (8, 64)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_per_role_dequant_equals_the_hip_blob_dequant(bits, gs, dtype):
    """`dequantize_packed_weight` (eager torch on the GPU, one role at a time) and the
    blob's one-launch HIP dequant give the same bits (tests/test_packed_expert_dequant.py:
    368-381)."""
    from vaayu_amd.moe_patch import (build_expert_blob, dequantize_expert_blob,
                                     dequantize_packed_weight)
    from vaayu_amd.synth import quantize_pack
    g = torch.Generator().manual_seed(bits + gs)
    by_role = {}
    for role, shape in (("gate", (768, 2048)), ("down", (2048, 768)), ("up", (768, 2048))):
        w = (torch.randn(shape, generator=g) * 0.02).bfloat16()
        packed, scale = quantize_pack(w, bits, gs, torch.float16)
        by_role[role] = {"weight_packed": packed.cuda(), "weight_scale": scale.cuda(),
                         "weight_shape": torch.tensor(list(shape))}
    via_hip = dequantize_expert_blob(build_expert_blob(by_role), dtype)
    for role, comps in by_role.items():
        assert torch.equal(dequantize_packed_weight(comps, dtype), via_hip[role]), role


def test_a_stream_off_16_bytes_takes_the_eager_path():
    """The kernel reads 16-byte units; a view starting one word in is dequantized by the
    eager arithmetic, with the same bits."""
    rng = np.random.default_rng(5)
    words = torch.from_numpy(rng.integers(-2 ** 31, 2 ** 31, 257, dtype=np.int64)
                             .astype(np.int32)).cuda()
    scale = torch.from_numpy(rng.uniform(0.001, 0.1, 257).astype(np.float32)).half().cuda()
    got = mp._hip_dequant(words[1:], scale[1:], 4, 8, torch.bfloat16)
    want = O.dequant_flat(words[1:].cpu(), scale[1:].cpu(), 4, 8, "bf16")
    assert np.array_equal(got.float().cpu().numpy(), want)
