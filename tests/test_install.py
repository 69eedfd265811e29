"""`install_packed_expert_kernels`: when the kernels are switched on at load, and when they
are (loudly or quietly) left off.

Ports the reference's installer cases (tests/test_packed_expert_install.py:22-232) onto a
stand-in engine: a tiny compressed-tensors checkpoint on disk, one safetensors shard per
MoE layer, indexed by this package's `ExpertOffsetIndex`, and namespace objects with the
fields the installer reads (vaayu/vaayu_base.py's model, its `_moe_blocks`). Cases that
need no kernel run on the CPU; the verdicts run the kernels on the GPU.
"""
import types

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F
from safetensors.torch import save_file

import vaayu_amd.moe_patch as mp
import vaayu_amd.packed_expert_kernels as pk
from vaayu_amd.expert_offset_index import ExpertOffsetIndex
from vaayu_amd.synth import quantize_pack

NUM_EXPERTS = 8
TOP_K = 2
gpu = pytest.mark.gpu


def _write_layer(root, layer, spec, hidden, inter, seed):
    """One MoE layer's shard. spec: {} packed int4 g32; {"group_size": 64} packed at
    another group size; None unquantized bf16 experts."""
    g = torch.Generator().manual_seed(seed)
    tensors = {}
    for e in range(NUM_EXPERTS):
        for name, shape in (("gate_proj", (inter, hidden)), ("down_proj", (hidden, inter)),
                            ("up_proj", (inter, hidden))):
            w = (torch.randn(shape, generator=g) * 0.05).bfloat16()
            key = f"{layer}.mlp.experts.{e}.{name}"
            if spec is None:
                tensors[f"{key}.weight"] = w
                continue
            packed, scale = quantize_pack(w, 4, spec.get("group_size", 32), torch.bfloat16)
            tensors[f"{key}.weight_packed"] = packed
            tensors[f"{key}.weight_scale"] = scale
            tensors[f"{key}.weight_shape"] = torch.tensor(list(shape))
    tensors[f"{layer}.mlp.gate.weight"] = torch.randn(NUM_EXPERTS, hidden, generator=g).bfloat16()
    save_file(tensors, str(root / f"{layer}.safetensors"))


def engine(tmp_path, *, device="cuda", hidden=256, inter=128, more_layers=(), act=None):
    """(vaayu_ref stand-in, its blocks): layer 0 packed int4 g32, then one layer per spec
    in `more_layers`."""
    specs = ({},) + tuple(more_layers)
    blocks = []
    for i, spec in enumerate(specs):
        name = f"model.layers.{i}"
        _write_layer(tmp_path, name, spec, hidden, inter, seed=i)
        experts = types.SimpleNamespace(act_fn=act if act is not None else nn.SiLU(),
                                        num_experts=NUM_EXPERTS)
        blocks.append(types.SimpleNamespace(
            forward_name="_make_fused_sparse_forward", layer_name=name, layer_idx=3 * i + 1,
            moe_module=types.SimpleNamespace(experts=experts), experts_attr="experts"))
    index = ExpertOffsetIndex(str(tmp_path))
    index.build(write_cache=False)
    ref = types.SimpleNamespace(running_device=device, running_dtype=torch.bfloat16,
                                _moe_blocks=blocks, _expert_offset_index=index,
                                checkpoint_path=str(tmp_path), moe_top_k=TOP_K)
    return ref, blocks


def _bare(**kw):
    base = dict(running_device="cuda", running_dtype=torch.bfloat16, _moe_blocks=[],
                _expert_offset_index=None, checkpoint_path="", moe_top_k=TOP_K)
    base.update(kw)
    return types.SimpleNamespace(**base)


@pytest.fixture
def fresh(monkeypatch):
    monkeypatch.setattr(pk, "_VERDICTS", {})
    monkeypatch.setattr(pk, "_PF_VERDICTS", {})


def _warnings(out):
    return [line for line in out.splitlines() if "WARNING" in line]


# ── CPU: nothing to install, refused before any kernel ──────────────────────────────────

def test_nothing_on_cpu():
    ref = _bare(running_device="cpu")
    assert pk.install_packed_expert_kernels(ref) is False
    assert not hasattr(ref, "_packed_moe_kernel")


def test_nothing_without_the_kernel_library(monkeypatch):
    monkeypatch.setattr(pk, "triton", None)
    assert pk.install_packed_expert_kernels(_bare()) is False


def test_nothing_without_a_fused_block():
    blocks = [types.SimpleNamespace(forward_name="_make_modulelist_sparse_forward")]
    assert pk.install_packed_expert_kernels(_bare(_moe_blocks=blocks,
                                                  _expert_offset_index=object())) is False


def test_nothing_without_an_offset_index():
    blocks = [types.SimpleNamespace(forward_name="_make_fused_sparse_forward")]
    assert pk.install_packed_expert_kernels(_bare(_moe_blocks=blocks)) is False


def test_another_gpu_is_refused_loudly(monkeypatch, capsys):
    monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)
    blocks = [types.SimpleNamespace(forward_name="_make_fused_sparse_forward")]
    ref = _bare(running_device="cuda:1", _moe_blocks=blocks, _expert_offset_index=object())
    assert pk.install_packed_expert_kernels(ref) is False
    out = capsys.readouterr().out
    assert "WARNING" in out and "not the current GPU" in out


def test_is_silu_judges_by_values():
    assert pk._is_silu(nn.SiLU(), "cpu", torch.bfloat16)
    assert pk._is_silu(F.silu, "cpu", torch.float32)
    assert not pk._is_silu(nn.GELU(), "cpu", torch.bfloat16)
    assert not pk._is_silu(None, "cpu", torch.bfloat16)
    assert not pk._is_silu(lambda t: 1 / 0, "cpu", torch.bfloat16)


def test_one_real_blob_reads_the_lowest_expert(tmp_path):
    """The blob the installer checks is expert 0's, built from the checkpoint's bytes."""
    ref, blocks = engine(tmp_path, device="cpu")
    blob = pk._one_real_blob(ref, blocks[0], "cpu")
    raw = {k: v for k, v in pk._read_expert_tensors(
        str(tmp_path / "model.layers.0.safetensors"),
        ref._expert_offset_index.index["model.layers.0"][0]).items()}
    want = mp.build_expert_blob(mp._group_packed_tensors_by_weight(raw))
    assert blob["geom"] == want["geom"] == (4, 32, (("gate", 128, 256), ("down", 256, 128),
                                                     ("up", 128, 256)))
    assert all(torch.equal(blob["flat"][k], want["flat"][k]) for k in ("packed", "scale"))


def test_one_real_blob_of_a_dense_layer_is_none_and_quiet(tmp_path, capsys):
    ref, blocks = engine(tmp_path, device="cpu", more_layers=(None,))
    assert pk._one_real_blob(ref, blocks[1], "cpu") is None
    assert "WARNING" not in capsys.readouterr().out


def test_one_real_blob_without_a_fused_pass_says_why(tmp_path, capsys, monkeypatch):
    ref, blocks = engine(tmp_path, device="cpu")
    monkeypatch.setattr(mp, "build_expert_blob", lambda by_role: None)
    assert pk._one_real_blob(ref, blocks[0], "cpu") is None
    assert "different bit widths or group sizes" in capsys.readouterr().out
    assert pk._one_real_blob(ref, blocks[0], "cpu", quiet=True) is None
    assert capsys.readouterr().out == ""


def test_prefill_eligibility_per_layer(tmp_path):
    """Eligibility from one real expert of each layer: a dense layer and one at another
    group size are left out, each with its reason; the size guard is the layer's own."""
    ref, blocks = engine(tmp_path, device="cpu", more_layers=(None, {"group_size": 64}, {}))
    blob = pk._one_real_blob(ref, blocks[0], "cpu")
    eligible, left_out = pk._prefill_eligibility(ref, blocks, blocks[0], blob, "cpu", 4 << 30)
    assert eligible == [blocks[0].layer_idx, blocks[3].layer_idx]
    assert left_out == {
        "experts not pack-quantized, or packed with no fused pass": [blocks[1].layer_idx],
        "a different geometry or scale dtype than the checked layer": [blocks[2].layer_idx]}
    held = NUM_EXPERTS * sum(t.numel() * t.element_size() for t in blob["flat"].values())
    blocks[3].moe_module.experts.num_experts = 2 * NUM_EXPERTS
    eligible, left_out = pk._prefill_eligibility(ref, blocks, blocks[0], blob, "cpu", 3 * held)
    assert eligible == [blocks[0].layer_idx]
    assert (f"one call can hold a layer's {2 * NUM_EXPERTS} experts on the GPU at once "
            f"({2 * held / 2**30:.2f} GiB)") in next(k for k in left_out if "one call" in k)


def test_describe_keeps_the_reference_wording():
    assert pk._describe((4, 128, ())) == "4-bit, group 128"
    assert pk._describe(("e4m3", (128, 128), ())) == "e4m3, scale block (128, 128)"


# ── GPU: the verdicts ─────────────────────────────────────────────────────────────────────

@gpu
def test_installs_on_a_packed_fused_block(tmp_path, capsys, fresh):
    ref, blocks = engine(tmp_path)
    assert pk.install_packed_expert_kernels(ref) is True
    bits, gs, _roles = ref._packed_moe_kernel
    assert (bits, gs) == (4, 32)
    out = capsys.readouterr().out
    assert "fused packed-expert decode kernel on 1 MoE layers (4-bit, group 32)" in out
    assert len(pk._VERDICTS) == 2, "fp32 and activation-dtype routing weights both checked"


@gpu
def test_a_non_silu_activation_is_left_alone(tmp_path, capsys, fresh):
    ref, _blocks = engine(tmp_path, act=nn.GELU())
    assert pk.install_packed_expert_kernels(ref) is False
    out = capsys.readouterr().out
    assert "not SiLU" in out and "WARNING" not in out
    assert not hasattr(ref, "_packed_moe_kernel")


@gpu
def test_a_dense_fused_checkpoint_is_left_alone(tmp_path, capsys, fresh):
    ref, blocks = engine(tmp_path, more_layers=(None,))
    ref._moe_blocks = blocks[1:]                 # only the unquantized layer
    assert pk.install_packed_expert_kernels(ref) is False
    assert "WARNING" not in capsys.readouterr().out
    assert not hasattr(ref, "_packed_moe_kernel")


@gpu
def test_a_disagreeing_kernel_is_refused_at_load(tmp_path, capsys, monkeypatch, fresh):
    monkeypatch.setattr(pk, "_launch", lambda x, pairs, w, out: out.zero_())
    ref, _blocks = engine(tmp_path)
    assert pk.install_packed_expert_kernels(ref) is False
    assert "WARNING" in capsys.readouterr().out
    assert not hasattr(ref, "_packed_moe_kernel")


@gpu
def test_installs_the_prefill_kernels_too(tmp_path, capsys, fresh):
    ref, blocks = engine(tmp_path)
    assert pk.install_packed_expert_kernels(ref) is True
    assert ref._packed_moe_prefill_kernel == frozenset({blocks[0].layer_idx})
    out = capsys.readouterr().out
    assert "fused packed-expert prefill kernel on 1 MoE layers (4-bit, group 32)" in out
    assert "WARNING" not in out
    assert len(pk._PF_VERDICTS) == 2, "fp32 and activation-dtype routing weights both checked"


@gpu
def test_a_disagreeing_prefill_kernel_keeps_the_decode_kernel(tmp_path, capsys, monkeypatch,
                                                               fresh):
    monkeypatch.setattr(pk, "_prefill_launch", lambda x, e, w, b, out, plan=None: out.zero_())
    ref, _blocks = engine(tmp_path)
    assert pk.install_packed_expert_kernels(ref) is True
    assert ref._packed_moe_kernel is not None
    assert not hasattr(ref, "_packed_moe_prefill_kernel")
    out = capsys.readouterr().out
    assert "prefill kernel refused" in out and "WARNING" in out


@gpu
def test_a_geometry_the_prefill_kernels_cannot_tile_keeps_the_decode_kernel(tmp_path, capsys,
                                                                            fresh):
    """hidden = intermediate = 64: the decode GEMV takes it, no MFMA K tile fits."""
    ref, _blocks = engine(tmp_path, hidden=64, inter=64)
    assert pk.install_packed_expert_kernels(ref) is True
    assert not hasattr(ref, "_packed_moe_prefill_kernel")
    out = capsys.readouterr().out
    assert "prefill kernel refused" in out and "K tile" in out


@gpu
def test_a_refused_decode_kernel_installs_no_prefill_kernel(tmp_path, monkeypatch, fresh):
    monkeypatch.setattr(pk, "_launch", lambda x, pairs, w, out: out.zero_())
    ref, _blocks = engine(tmp_path)
    assert pk.install_packed_expert_kernels(ref) is False
    assert not hasattr(ref, "_packed_moe_prefill_kernel")


@gpu
def test_layers_too_large_to_hold_at_once_keep_the_per_expert_prefill(tmp_path, capsys,
                                                                      monkeypatch, fresh):
    """Every layer over half the prefill headroom: one WARNING with the derived size, no
    prefill verdict taken, the decode kernel unaffected."""
    ref, _blocks = engine(tmp_path, more_layers=({},))
    monkeypatch.setattr(pk, "_PREFILL_VRAM_HEADROOM", 64 * 1024)
    assert pk.install_packed_expert_kernels(ref) is True
    assert ref._packed_moe_kernel is not None
    assert not hasattr(ref, "_packed_moe_prefill_kernel")
    warnings = _warnings(capsys.readouterr().out)
    assert len(warnings) == 1
    assert ("prefill kernel not installed: one call can hold a layer's 8 experts"
            in warnings[0])
    assert warnings[0].endswith("prefill headroom; prefill keeps the per-expert path")
    assert pk._PF_VERDICTS == {}, "refused before the kernels ran"


@gpu
@pytest.mark.parametrize("second, why", [
    (None, "not pack-quantized"),
    ("no-fused-pass", "no fused pass"),
    ({"group_size": 64}, "a different geometry or scale dtype"),
], ids=["unquantized", "no-fused-pass", "another-group-size"])
def test_a_layer_the_prefill_kernels_cannot_take_is_left_out_and_named(tmp_path, capsys,
                                                                       monkeypatch, fresh,
                                                                       second, why):
    if second == "no-fused-pass":
        second = {}
        real, calls = mp.build_expert_blob, []

        def build(by_role):                  # every expert after the first has no fused pass
            calls.append(1)
            return real(by_role) if len(calls) == 1 else None
        monkeypatch.setattr(mp, "build_expert_blob", build)
    ref, blocks = engine(tmp_path, more_layers=(second,))
    first, other = (b.layer_idx for b in blocks)
    assert pk.install_packed_expert_kernels(ref) is True
    assert ref._packed_moe_prefill_kernel == frozenset({first})
    assert ref._packed_moe_kernel is not None
    out = capsys.readouterr().out
    assert "fused packed-expert prefill kernel on 1 MoE layers (4-bit, group 32)" in out
    warnings = _warnings(out)
    assert len(warnings) == 1
    assert (f"prefill kernel not used on 1 of 2 MoE layers (layer indices {other}): "
            in warnings[0]) and why in warnings[0]
    assert warnings[0].endswith("prefill keeps the per-expert path there")
    assert "decode kernel not installed" not in out, "the probe of the other layer is quiet"


@gpu
def test_layers_left_out_for_different_reasons_share_one_warning(tmp_path, capsys, fresh):
    ref, blocks = engine(tmp_path, more_layers=(None, {"group_size": 64}))
    first, dense, other = (b.layer_idx for b in blocks)
    assert pk.install_packed_expert_kernels(ref) is True
    assert ref._packed_moe_prefill_kernel == frozenset({first})
    warnings = _warnings(capsys.readouterr().out)
    assert len(warnings) == 1
    assert warnings[0].endswith(
        f"not used on 2 of 3 MoE layers (layer indices {dense}, {other}): experts not "
        f"pack-quantized, or packed with no fused pass (layers {dense}); a different geometry "
        f"or scale dtype than the checked layer (layers {other}); prefill keeps the "
        f"per-expert path there")


@gpu
def test_a_layer_with_more_experts_than_fit_is_left_out_with_its_size(tmp_path, capsys,
                                                                      monkeypatch, fresh):
    ref, blocks = engine(tmp_path, more_layers=({},))
    small, large = blocks
    blob = pk._one_real_blob(ref, small, "cuda")
    held = NUM_EXPERTS * sum(t.numel() * t.element_size() for t in blob["flat"].values())
    large.moe_module.experts.num_experts = 2 * NUM_EXPERTS
    monkeypatch.setattr(pk, "_PREFILL_VRAM_HEADROOM", 3 * held)     # half: 1.5x one layer
    assert pk.install_packed_expert_kernels(ref) is True
    assert ref._packed_moe_prefill_kernel == frozenset({small.layer_idx})
    warnings = _warnings(capsys.readouterr().out)
    assert len(warnings) == 1
    assert (f"not used on 1 of 2 MoE layers (layer indices {large.layer_idx}): one call can "
            f"hold a layer's {2 * NUM_EXPERTS} experts on the GPU at once "
            f"({2 * held / 2**30:.2f} GiB)") in warnings[0]
