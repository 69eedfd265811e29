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
