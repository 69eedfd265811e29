"""FP8 block-scaled and microscaled (MX) expert weight formats.

Mirrors of the reference's two dequant entry points for these formats, same signatures and
results:

  dequantize_block_scaled(weight, scale, dtype)        vaayu/model_code/deepseek_v4/
      modeling_deepseek_v4.py:228-240 -- float8_e4m3fn weight, one scale per (bo x bi)
      tile, bo and bi derived from the two shapes.
  upcast_from_mxfp(tensor, scale, target_dtype, axis)  vendor gpt_oss_triton_kernels
      numerics_details/mxfp.py:256-299 (`upcast_from_mxfp_torch`) and its Triton twin
      mxfp_details/_upcast_from_mxfp.py -- e2m1 (two per uint8, even element in the low
      nibble) or e4m3 codes, one e8m0 scale per 32 elements along `axis`.

For CUDA tensors the work is one HIP kernel (vaayu_dequant_fp8_block / vaayu_upcast_mx in
libvaayu_amd.so), bit-exact with the reference arithmetic: the fp32 product rounded once,
then one rounding to the output dtype. A scale byte 0xFF gives NaN (the Triton twin's rule);
0 gives 0 (the fp32 with exponent bits 0). Without the library a CUDA call raises
ImportError. CPU tensors take the reference's own eager arithmetic, as the reference does on
the CPU.
"""
import torch

from . import _lib

_OUT_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}
_E8M0 = getattr(torch, "float8_e8m0fnu", None)
_MX_E2M1, _MX_E4M3 = 0, 1


def _scale_code(scale: torch.Tensor) -> int:
    if scale.dtype in (torch.bfloat16, torch.float16, torch.float32):
        return _OUT_CODE[scale.dtype]
    if scale.dtype == torch.uint8 or (_E8M0 is not None and scale.dtype == _E8M0):
        return 3
    raise TypeError(f"block scale dtype {scale.dtype} (bf16, fp16, fp32 or e8m0)")


def _e8m0_fp32(scale_u8: torch.Tensor) -> torch.Tensor:
    """2^(s - 127) as the fp32 with exponent bits s; 0xFF is NaN."""
    f = (scale_u8.to(torch.int32) << 23).view(torch.float32)
    return torch.where(scale_u8 == 0xFF, torch.full_like(f, float("nan")), f)


def dequantize_block_scaled(weight: torch.Tensor, scale: torch.Tensor,
                            dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Multiply a block-scaled float8_e4m3fn weight out into `dtype`: `scale[i, j]` covers
    `weight[i*bo:(i+1)*bo, j*bi:(j+1)*bi]`, bo and bi derived from the shapes
    (vaayu/model_code/deepseek_v4/modeling_deepseek_v4.py:228-240)."""
    if weight.dim() != 2 or scale.dim() != 2:
        raise ValueError("dequantize_block_scaled takes a 2-D weight and a 2-D scale grid")
    rows, cols = weight.shape
    if rows % scale.shape[0] or cols % scale.shape[1]:
        raise ValueError(f"scale grid {tuple(scale.shape)} does not tile weight {tuple(weight.shape)}")
    if dtype not in _OUT_CODE:
        raise TypeError(f"output dtype {dtype}")
    if weight.device.type != "cuda":
        bo, bi = rows // scale.shape[0], cols // scale.shape[1]
        s = _e8m0_fp32(scale.view(torch.uint8)) if _scale_code(scale) == 3 else scale.float()
        tiled = weight.unflatten(0, (-1, bo)).unflatten(-1, (-1, bi)).float() * s[:, None, :, None]
        return tiled.flatten(2, 3).flatten(0, 1).to(dtype)
    lib = _lib.load()
    w = weight.contiguous().view(torch.uint8)
    sc = scale.contiguous()
    code = _scale_code(sc)
    if code == 3:
        sc = sc.view(torch.uint8)
    out = torch.empty(rows, cols, dtype=dtype, device=weight.device)
    rc = lib.vaayu_dequant_fp8_block(w.data_ptr(), sc.data_ptr(), code, out.data_ptr(),
                                     _OUT_CODE[dtype], rows, cols, sc.shape[0], sc.shape[1],
                                     _lib.stream_ptr(weight.device))
    _lib.check(rc, "vaayu_dequant_fp8_block")
    return out


def cvt_e2m1_to_fp32(input_tensor: torch.Tensor) -> torch.Tensor:
    """uint8 [..., n] of e2m1 pairs -> fp32 [..., 2n], even element from the low nibble
    (vendor …/numerics_details/mxfp.py:238-253)."""
    if input_tensor.dtype != torch.uint8:
        raise TypeError("e2m1 codes come packed in uint8")
    t = input_tensor.to(torch.int32)
    table = torch.tensor([0.0, 0.5, 1, 1.5, 2, 3, 4, 6], dtype=torch.float32, device=t.device)
    table = torch.cat([table, -table])
    out = torch.stack([table[t & 0xF], table[(t >> 4) & 0xF]], dim=-1)
    return out.view(*input_tensor.shape[:-1], -1)


def upcast_from_mxfp(tensor: torch.Tensor, scale: torch.Tensor, target_dtype: torch.dtype,
                     axis: int) -> torch.Tensor:
    """MX codes along `axis` times 2^(s - 127) per 32 elements, in `target_dtype`
    (vendor …/numerics_details/mxfp.py:256-299). `tensor`: uint8 (e2m1 pairs along `axis`)
    or float8_e4m3fn; `scale`: uint8 / float8_e8m0fnu exponents. The result is laid out
    like the reference's: computed with `axis` last, then transposed back (a view)."""
    ndim = tensor.ndim
    if not -ndim <= axis < ndim:
        raise ValueError(f"invalid axis {axis}")
    if tensor.dtype == torch.uint8:
        fmt = _MX_E2M1
    elif tensor.dtype == torch.float8_e4m3fn:
        fmt = _MX_E4M3
    else:
        raise TypeError(f"MX codes of dtype {tensor.dtype} (uint8 e2m1 pairs or float8_e4m3fn)")
    if target_dtype not in _OUT_CODE:
        raise TypeError(f"target dtype {target_dtype}")
    axis = axis % ndim
    t = tensor.transpose(axis, ndim - 1)
    s = scale.transpose(axis, scale.ndim - 1)
    if s.dtype != torch.uint8:
        s = s.view(torch.uint8)
    k = t.shape[-1] * (2 if fmt == _MX_E2M1 else 1)
    if s.shape[-1] != (k + 31) // 32 or s.shape[:-1] != t.shape[:-1]:
        raise ValueError(f"scale shape {tuple(scale.shape)} does not match codes {tuple(tensor.shape)}")
    if t.device.type != "cuda":
        vals = cvt_e2m1_to_fp32(t) if fmt == _MX_E2M1 else t.to(torch.float32)
        f = _e8m0_fp32(s).repeat_interleave(32, dim=-1)[..., :k]
        out = (vals * f).to(target_dtype).contiguous()
        return out.transpose(axis, ndim - 1)
    lib = _lib.load()
    lead = t.shape[:-1]
    rows = 1
    for d in lead:
        rows *= d
    tq = t.contiguous().view(torch.uint8).reshape(rows, -1)
    ts = s.contiguous().reshape(rows, -1)
    out = torch.empty(*lead, k, dtype=target_dtype, device=tensor.device)
    rc = lib.vaayu_upcast_mx(tq.data_ptr(), fmt, ts.data_ptr(), out.data_ptr(),
                             _OUT_CODE[target_dtype], rows, k, _lib.stream_ptr(tensor.device))
    _lib.check(rc, "vaayu_upcast_mx")
    return out.transpose(axis, ndim - 1)


upcast_from_mxfp_torch = upcast_from_mxfp


# ── FP8 / MXFP4 expert blobs ────────────────────────────────────────────────────────────
#
# The reference keeps packed experts as {"flat": {"packed", "scale"}, "geom": (bits, gs,
# roles)} (vaayu/moe_patch.py:794-846). FP8 and MXFP4 experts use the same container: the
# roles gate, down, up concatenated, codes along the last dim in int32 words, and geom
#   ("e4m3", (bo, bi), roles)  float8_e4m3fn codes, one fp32 scale per bo x bi tile
#   ("mxfp4", 32, roles)       e2m1 codes (even element in the low nibble), one E8M0 byte
#                              per 32 codes along a row
# so the pointer tables, layout arithmetic and kernels take them like the int blobs.

FMT_INT, FMT_E4M3, FMT_MXFP4 = 0, 1, 2


def geom_format(geom):
    """(format code, code bits, codes per scale along a row, rows per scale) of a blob
    geometry."""
    kind, gs, _roles = geom
    if kind == "e4m3":
        bo, bi = gs
        return FMT_E4M3, 8, int(bi), int(bo)
    if kind == "mxfp4":
        return FMT_MXFP4, 4, 32, 1
    return FMT_INT, int(kind), int(gs), 1


def blob_layout(geom) -> dict:
    """{role: (word offset, scale offset, rows, cols)} in the flat streams, for every
    format (the int case is the reference's `_layout`, vaayu/packed_expert_kernels.py:301-309)."""
    _fmt, bits, group, brows = geom_format(geom)
    out, w_at, s_at = {}, 0, 0
    for role, rows, cols in geom[2]:
        out[role] = (w_at, s_at, rows, cols)
        w_at += rows * cols * bits // 32
        s_at += (rows // brows) * (cols // group)
    return out


def _fp8_codes(w: torch.Tensor, block) -> tuple:
    """(e4m3 codes, fp32 scales) of one role: scale = amax / 448 per block (1 for an
    all-zero block), codes = the e4m3 cast of w / scale."""
    bo, bi = block
    rows, cols = w.shape
    t = w.float().reshape(rows // bo, bo, cols // bi, bi)
    amax = t.abs().amax(dim=(1, 3))
    scale = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    q = (t / scale[:, None, :, None]).reshape(rows, cols).to(torch.float8_e4m3fn)
    return q, scale.float()


_E2M1_GRID = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def _mxfp4_codes(w: torch.Tensor) -> tuple:
    """(e2m1 codes as uint8 pairs [rows, cols/2], E8M0 scales [rows, cols/32]) of one role:
    per 32 along a row, the scale exponent makes the block's amax at most 6, each value
    rounded to the nearest e2m1 magnitude (ties to the even code)."""
    rows, cols = w.shape
    t = w.float().reshape(rows, cols // 32, 32)
    amax = t.abs().amax(dim=-1)
    e = torch.where(amax > 0, torch.ceil(torch.log2(amax / 6.0)), torch.full_like(amax, -127))
    e = e.clamp(-127, 127)
    scale = torch.pow(2.0, e)
    v = (t / scale[..., None]).clamp(-6.0, 6.0)
    grid = _E2M1_GRID.to(v.device)
    mag = (v.abs()[..., None] - grid).abs()
    best = mag.argmin(dim=-1)                                   # lowest code on ties
    code = best + torch.where(v < 0, 8, 0)
    code = torch.where(best == 0, torch.zeros_like(code), code)  # -0 stored as +0
    code = code.reshape(rows, cols).to(torch.uint8)
    packed = (code[:, 0::2] | (code[:, 1::2] << 4)).to(torch.uint8)
    return packed, (e + 127).to(torch.uint8)


def random_format_expert(fmt: str, hidden: int, inter: int, *, generator, device,
                         std: float = 0.02) -> dict:
    """A synthetic FP8 ("e4m3", 128 x 128 fp32 block scales) or MXFP4 ("mxfp4") expert blob
    of bf16 N(0, std) weights, roles gate, down, up."""
    roles = (("gate", inter, hidden), ("down", hidden, inter), ("up", inter, hidden))
    packed, scales = [], []
    for _role, rows, cols in roles:
        w = (torch.randn(rows, cols, generator=generator, device=device) * std).to(torch.bfloat16)
        if fmt == "e4m3":
            q, s = _fp8_codes(w, (128, 128))
            packed.append(q.view(torch.uint8).reshape(-1))
        elif fmt == "mxfp4":
            q, s = _mxfp4_codes(w)
            packed.append(q.reshape(-1))
        else:
            raise ValueError(f"format {fmt}")
        scales.append(s.reshape(-1))
    words = torch.cat(packed).contiguous().view(torch.int32)
    geom = ("e4m3", (128, 128), roles) if fmt == "e4m3" else ("mxfp4", 32, roles)
    return {"flat": {"packed": words, "scale": torch.cat(scales).contiguous()}, "geom": geom}


def dequantize_format_blob(blob: dict, dtype: torch.dtype) -> dict:
    """{role: dense weight} of an FP8 / MXFP4 blob: each role through the mirrors above
    (HIP on a GPU, the reference's arithmetic on the CPU)."""
    fmt, _bits, group, brows = geom_format(blob["geom"])
    lay = blob_layout(blob["geom"])
    codes = blob["flat"]["packed"].view(torch.uint8)
    scale = blob["flat"]["scale"]
    out = {}
    for role, (w_at, s_at, rows, cols) in lay.items():
        if fmt == FMT_E4M3:
            q = codes[w_at * 4: w_at * 4 + rows * cols].view(rows, cols)
            sc = scale[s_at: s_at + (rows // brows) * (cols // group)].view(rows // brows, cols // group)
            out[role] = dequantize_block_scaled(q.view(torch.float8_e4m3fn), sc, dtype)
        else:
            q = codes[w_at * 4: w_at * 4 + rows * cols // 2].view(rows, cols // 2)
            sc = scale[s_at: s_at + rows * cols // 32].view(rows, cols // 32)
            out[role] = upcast_from_mxfp(q, sc, dtype, axis=-1)
    return out
