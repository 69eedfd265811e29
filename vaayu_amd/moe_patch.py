"""The packed-format half of Vaayu's MoE layer, with the dequant on a HIP kernel.

Same names, arguments, results and errors as the functions of the reference module
`vaayu/moe_patch.py` that the packed-expert path uses, so the engine's expert cache, fused
forward and prefill stager can call these unchanged:

  checkpoint keys -> roles     `_group_packed_tensors_by_weight`   (moe_patch.py:532-551)
  unpack / per-role dequant    `unpack_int32_to_int8`, `dequantize_packed_weight` (:668-744)
  one expert as one blob       `build_expert_blob`                  (:794-846)
  blob -> dense weights        `_fused_dequant_kernel`, `dequantize_expert_blob`,
                               `expert_weights_from_entry`          (:750-891)
  fixed-order accumulate       `accumulate_expert_outputs`          (:914-940)
  shared expert                `_shared_expert_output`              (:554-580)
  routing                      `route_experts`, `truncate_top_k`, `_routing_to_host`
                                                                    (:130-243)

What differs is where the work runs: on a GPU tensor the whole-blob dequant is the HIP
kernel `vaayu_dequant_blob` (bit-exact with the eager arithmetic; the reference compiles
the eager function with torch.compile instead). On the CPU, and for dtypes the kernel
does not produce (float64), the eager torch arithmetic runs, as in the reference.
"""
from __future__ import annotations

import torch

from . import _lib

# Checkpoint key substrings -> expert roles (the Mixtral and DeepSeek/Qwen spellings).
_EXPERT_WEIGHT_ROLES: list = [
    (".w1.", "gate"), (".w2.", "down"), (".w3.", "up"),
    (".gate_proj.", "gate"), (".down_proj.", "down"), (".up_proj.", "up"),
]

# The tensors a compressed-tensors `pack-quantized` linear is stored as.
_PACKED_COMPONENT_KEYS = {
    "weight_packed", "weight_scale", "weight_shape", "weight_zero_point", "weight_g_idx",
}

_ASYMMETRIC = ("asymmetric / act-order pack-quantized experts carry a zero point or g_idx "
               "that is not applied here; this checkpoint would decode to shifted weights. "
               "Supported: symmetric group quantization.")


def _role_of(key: str):
    for pattern, role in _EXPERT_WEIGHT_ROLES:
        if pattern in key:
            return role
    return None


def _group_packed_tensors_by_weight(raw: dict) -> dict:
    """{"gate": {component: tensor}, "down": ..., "up": ...} of one expert's packed tensors.
    An expert that is not packed gives three empty dicts."""
    out = {"gate": {}, "down": {}, "up": {}}
    for key, tensor in raw.items():
        role = _role_of(key)
        if role is None:
            continue
        component = key.rsplit(".", 1)[-1]
        if component in _PACKED_COMPONENT_KEYS:
            out[role][component] = tensor
    return out


def _packed_roles_complete(packed: dict) -> bool:
    """Each role has both its codes and its scales."""
    return all({"weight_packed", "weight_scale"} <= set(packed[r]) for r in ("gate", "down", "up"))


def _upload_packed_expert(packed: dict, device, timing: dict = None) -> dict:
    """Device copies of one packed expert's components; `weight_shape` stays on the host."""
    return {r: {k: (v if k == "weight_shape" else v.to(device, non_blocking=True))
                for k, v in packed[r].items()}
            for r in ("gate", "down", "up")}


def unpack_int32_to_int8(packed: torch.Tensor, num_bits: int, cols: int) -> torch.Tensor:
    """Signed int8 codes [rows, cols] from compressed-tensors int32 words.

    A row is one little-endian bit stream: code i sits at bits [i*num_bits, (i+1)*num_bits)
    and is stored unsigned with offset 2^(num_bits-1)."""
    rows, n_words = packed.shape
    offset = 1 << (num_bits - 1)
    mask = (1 << num_bits) - 1
    if 32 % num_bits == 0:
        per = 32 // num_bits
        shifts = torch.arange(per, device=packed.device, dtype=torch.int32) * num_bits
        codes = (packed.unsqueeze(-1) >> shifts) & mask
        return (codes.reshape(rows, n_words * per)[:, :cols] - offset).to(torch.int8)
    # Codes straddle words: gather each code's low part from its word and the rest from
    # the next one. 32 codes fill exactly `num_bits` words.
    if n_words % num_bits:
        packed = torch.nn.functional.pad(packed, (0, num_bits - n_words % num_bits))
    blocks = packed.reshape(-1, num_bits)
    start = torch.arange(32, device=packed.device, dtype=torch.int64) * num_bits
    word, bit = start // 32, (start % 32).to(torch.int32)
    low_bits = torch.clamp(32 - bit, max=num_bits)
    vals = (blocks[:, word] >> bit) & ((1 << low_bits) - 1)
    spill = low_bits < num_bits
    if bool(spill.any()):
        high = num_bits - low_bits[spill]
        vals[:, spill] |= (blocks[:, word[spill] + 1] & ((1 << high) - 1)) << low_bits[spill]
    return (vals.reshape(rows, -1)[:, :cols] - offset).to(torch.int8)


def dequantize_packed_weight(components: dict, dtype: torch.dtype) -> torch.Tensor:
    """One packed linear's dense weight. Bit width and group size come from the tensors:
    bits = words*32 / (rows*cols), group = cols / scale.shape[-1]."""
    if "weight_zero_point" in components or "weight_g_idx" in components:
        raise NotImplementedError(_ASYMMETRIC)
    packed, scale = components["weight_packed"], components["weight_scale"]
    rows, cols = (int(v) for v in components["weight_shape"].tolist())
    bits, rem = divmod(packed.numel() * 32, rows * cols)
    if rem or not 1 <= bits <= 8:
        raise ValueError(f"cannot derive bit width: {packed.numel()} int32 words for a "
                         f"{rows}x{cols} weight")
    codes = unpack_int32_to_int8(packed, bits, cols)
    groups = scale.shape[-1]
    return (codes.view(rows, groups, cols // groups).to(dtype)
            * scale.view(rows, groups, 1).to(dtype)).view(rows, cols)


def _fused_dequant_kernel(flat_packed, flat_scale, num_bits, group_size, dtype):
    """The whole flat code stream of one expert, unpacked and scaled: codes in `dtype`
    minus 2^(bits-1), times the group's scale in `dtype` (eager torch, any device)."""
    per = 32 // num_bits
    shifts = torch.arange(per, device=flat_packed.device, dtype=torch.int32) * num_bits
    codes = (flat_packed.unsqueeze(-1) >> shifts) & ((1 << num_bits) - 1)
    codes = codes.view(-1, group_size).to(dtype) - (1 << (num_bits - 1))
    return (codes * flat_scale.reshape(-1, 1).to(dtype)).view(-1)


def _hip_dequant(flat_packed, flat_scale, num_bits, group_size, dtype):
    """`_fused_dequant_kernel` on the GPU: one HIP launch, the same bits. The kernel reads
    codes in 16-byte units; a stream that does not start on 16 bytes takes the eager path."""
    packed = flat_packed.contiguous()
    scale = flat_scale.contiguous()
    if packed.data_ptr() % 16:
        return _fused_dequant_kernel(packed, scale, num_bits, group_size, dtype)
    lib = _lib.load()
    out = torch.empty(flat_packed.numel() * (32 // num_bits), dtype=dtype,
                      device=flat_packed.device)
    rc = lib.vaayu_dequant_blob(packed.data_ptr(), scale.data_ptr(),
                                _lib.DTYPE_CODE[scale.dtype], out.data_ptr(),
                                _lib.DTYPE_CODE[dtype], packed.numel(), num_bits, group_size,
                                _lib.stream_ptr(packed.device))
    _lib.check(rc, "vaayu_dequant_blob")
    return out


def _fused_dequant_fn(num_bits, group_size, dtype, device_type):
    """The blob dequant for this device: the HIP kernel on a GPU for the dtypes it
    writes, the eager arithmetic otherwise."""
    if device_type == "cuda" and dtype in _lib.DTYPE_CODE and 32 % num_bits == 0:
        return _hip_dequant
    return _fused_dequant_kernel


def build_expert_blob(by_role: dict) -> "dict | None":
    """One expert's packed roles as one blob {"flat": {"packed", "scale"}, "geom"}, or
    None when the roles cannot share one flat stream (not packed, or different bit
    widths / group sizes, or codes straddling words). Roles keep the dict's order;
    geom = (bits, group, ((role, rows, cols), ...)). A zero point or g_idx raises."""
    geom = []
    for role, comps in by_role.items():
        if "weight_zero_point" in comps or "weight_g_idx" in comps:
            raise NotImplementedError(_ASYMMETRIC)
        if not {"weight_packed", "weight_scale", "weight_shape"} <= set(comps):
            return None
        rows, cols = (int(v) for v in comps["weight_shape"].tolist())
        bits, rem = divmod(comps["weight_packed"].numel() * 32, rows * cols)
        gs = cols // comps["weight_scale"].shape[-1]
        geom.append((role, rows, cols, bits, gs, rem))
    if not geom:
        return None
    bits, gs = geom[0][3], geom[0][4]
    if not bits or 32 % bits:
        return None
    for _role, _rows, cols, b, g, rem in geom:
        if rem or b != bits or g != gs or cols % (32 // bits):
            return None
    roles = [g[0] for g in geom]
    return {
        "flat": {
            "packed": torch.cat([by_role[r]["weight_packed"].reshape(-1) for r in roles]),
            "scale": torch.cat([by_role[r]["weight_scale"].reshape(-1) for r in roles]),
        },
        "geom": (bits, gs, tuple((g[0], g[1], g[2]) for g in geom)),
    }


def dequantize_expert_blob(blob: dict, dtype: torch.dtype) -> dict:
    """{role: dense weight} from a blob: one dequant over the flat stream, then views
    (FP8 / MXFP4 blobs: their per-role dequant)."""
    if isinstance(blob["geom"][0], str):
        from .block_formats import dequantize_format_blob
        return dequantize_format_blob(blob, dtype)
    bits, gs, roles = blob["geom"]
    packed, scale = blob["flat"]["packed"], blob["flat"]["scale"]
    flat = _fused_dequant_fn(bits, gs, dtype, packed.device.type)(packed, scale, bits, gs, dtype)
    out, at = {}, 0
    for role, rows, cols in roles:
        out[role] = flat[at:at + rows * cols].view(rows, cols)
        at += rows * cols
    return out


def expert_weights_from_entry(entry: dict, dtype: torch.dtype) -> tuple:
    """(w_gate, w_down, w_up) of a cached expert: a dense entry as stored, a blob
    dequantized."""
    dense = entry["dense"] if "dense" in entry else dequantize_expert_blob(entry, dtype)
    return dense["gate"], dense["down"], dense["up"]


def dequantize_expert_weights(by_role: dict, dtype: torch.dtype) -> dict:
    """{role: dense weight}: one pass over a blob when the roles make one, else per role."""
    blob = build_expert_blob(by_role)
    if blob is None:
        return {role: dequantize_packed_weight(c, dtype) for role, c in by_role.items()}
    return dequantize_expert_blob(blob, dtype)


def accumulate_expert_outputs(final_hidden, contributions) -> None:
    """Add each (expert id, token rows, values) contribution into `final_hidden` in
    ascending expert id, whatever order they arrived in: fp32 addition does not
    associate, so only a fixed order makes the layer a function of its input."""
    for _e, token_idx, hidden in sorted(contributions, key=lambda c: c[0]):
        final_hidden.index_add_(0, token_idx, hidden.to(final_hidden.dtype))


def _shared_expert_output(moe_mod, flat_hidden):
    """The block's always-on shared expert on `flat_hidden`, or None: a child whose name
    holds "shared_expert" is the expert; one ending in "_gate" is a sigmoid gate over it
    (Qwen2 / Qwen3-Next); without a gate it is added as is (DeepSeek)."""
    shared = gate = None
    for name, child in moe_mod.named_children():
        if "shared_expert" not in name:
            continue
        if name.endswith("_gate"):
            gate = child
        elif shared is None:
            shared = child
    if shared is None:
        return None
    out = shared(flat_hidden)
    return torch.sigmoid(gate(flat_hidden)) * out if gate is not None else out


def unique_expert_indices(expert_indices_cpu) -> list:
    """Routed expert ids over every position, ascending, each once."""
    return sorted(int(v) for v in expert_indices_cpu.flatten().unique().tolist())


def route_experts(moe_module, router_logits, top_k: int):
    """(weights, indices) of one layer: the model's `route_tokens_to_experts` when it has
    one (indices told from weights by dtype, leading dims restored), else softmax of the
    fp32 logits, top-k, renormalised."""
    fn = getattr(moe_module, "route_tokens_to_experts", None)
    if not callable(fn):
        w, idx = torch.topk(router_logits.float().softmax(dim=-1), top_k, dim=-1)
        return w / w.sum(dim=-1, keepdim=True), idx
    lead = router_logits.shape[:-1]
    a, b = fn(router_logits.reshape(-1, router_logits.shape[-1]))
    idx, w = (a, b) if not a.is_floating_point() else (b, a)
    return w.reshape(*lead, -1), idx.reshape(*lead, -1)


def truncate_top_k(weights, indices, k, p=None):
    """Decode-time expert budget on routed (weights, indices); shapes unchanged.

    `k`: keep the k largest weights. `p`: keep per row the fewest slots whose normalised
    weight reaches p, re-pointing each dropped slot at the row's top-1 expert with weight
    0. Kept weights are rescaled to the row's original sum (snapped to exactly 1 when it
    is 1 within 1e-2). With neither budget active the SAME tensors are returned."""
    n = weights.shape[-1]
    if (k is None or k >= n) and p is None:
        return weights, indices
    total = weights.float().sum(dim=-1, keepdim=True)
    total = torch.where((total - 1.0).abs() < 1e-2, torch.ones_like(total), total)
    if k is not None and k < n:
        w, pos = torch.topk(weights.float(), k, dim=-1)
        weights = (w / w.sum(dim=-1, keepdim=True) * total).to(weights.dtype)
        indices = indices.gather(-1, pos)
    if p is None:
        return weights, indices
    w = weights.float()
    w = w / w.sum(dim=-1, keepdim=True)
    ws, order = torch.sort(w, dim=-1, descending=True)
    keep = torch.zeros_like(ws, dtype=torch.bool).scatter(-1, order, (ws.cumsum(-1) - ws) < p)
    top1 = indices.gather(-1, order[..., :1]).expand_as(indices)
    w = torch.where(keep, w, torch.zeros_like(w))
    w = w / w.sum(dim=-1, keepdim=True) * total
    return w.to(weights.dtype), torch.where(keep, indices, top1)


def _routing_to_host(expert_indices):
    """(ids on the host, the routed ids ascending) through one device-to-host copy."""
    cpu = expert_indices.cpu()
    if cpu.numel() <= cpu.shape[-1]:
        return cpu, sorted(set(cpu.reshape(-1).tolist()))
    return cpu, cpu.unique().tolist()
