"""Where every expert's tensors sit inside a checkpoint's safetensors shards, and loading a
layer's experts from those byte ranges straight into HBM-resident blobs.

`ExpertOffsetIndex` is the drop-in for Vaayu's `vaayu/persist/expert_offset_index.py:41-333`
(same constructor, `build` / `load_cached` / `build_or_load`, `index`,
`fused_layer_tensors`, `get_expert_offsets`, `moe_layer_names`, the guard that refuses an
empty index for an MoE config, and the same JSON cache file, version 2 written and
version 1 read). Two layouts are recognised by their keys and shapes, never by model name:

  per-expert  keys with an `.experts.<N>.` component, one tensor per expert (Mixtral,
              DeepSeek, Qwen MoE, and compressed-tensors AWQ / GPTQ checkpoints, whose
              `weight_packed` / `weight_scale` / `weight_shape` keys are per expert)
  fused       one tensor per layer under an `experts.` prefix whose leading axis is the
              config's expert count (gpt-oss): expert i is the i-th contiguous byte range.

`load_expert_tensors` reads one expert's tensors with as few reads as the byte ranges
allow; `load_resident_experts` puts a whole layer of compressed-tensors experts on the GPU
as the blobs the packed-expert kernels take (vaayu/moe_patch.py:527-580 groups the keys by
role, `build_expert_blob` concatenates the roles), staging each expert through pinned host
memory with one host-to-device copy.
"""
from __future__ import annotations

import json
import re
import struct
from dataclasses import dataclass
from pathlib import Path

import torch

_EXPERT_RE = re.compile(r"\.experts\.(\d+)\.")
_FUSED_EXPERTS_RE = re.compile(r"\.experts\.[A-Za-z_][A-Za-z0-9_]*$")
_SHARD_RE = re.compile(r"-(\d{5})-of-(\d{5})\.safetensors$")

# safetensors dtype names -> torch dtypes
SAFETENSORS_DTYPES = {
    "F64": torch.float64, "F32": torch.float32, "F16": torch.float16, "BF16": torch.bfloat16,
    "I64": torch.int64, "I32": torch.int32, "I16": torch.int16, "I8": torch.int8,
    "U8": torch.uint8, "BOOL": torch.bool, "F8_E4M3": torch.float8_e4m3fn,
    "F8_E5M2": torch.float8_e5m2,
}


@dataclass
class ExpertTensorMeta:
    file_offset: int   # absolute byte offset from the start of the file
    byte_length: int
    shape: list
    dtype: str         # the safetensors dtype name, e.g. "BF16"


def _meta_to_raw(m: ExpertTensorMeta) -> dict:
    return {"file_offset": m.file_offset, "byte_length": m.byte_length, "shape": m.shape,
            "dtype": m.dtype}


def _raw_to_meta(r: dict) -> ExpertTensorMeta:
    return ExpertTensorMeta(r["file_offset"], r["byte_length"], r["shape"], r["dtype"])


def read_header(shard_path) -> tuple:
    """(header dict, byte offset where the tensor data starts) of one safetensors file."""
    with open(shard_path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        return json.loads(f.read(n)), 8 + n


def assert_checkpoint_complete(checkpoint_dir) -> None:
    """RuntimeError when a sharded checkpoint is missing shards, by its file names
    (`-0000i-of-0000n`) or by its `model.safetensors.index.json` weight map
    (vaayu/persist/checkpoint_integrity.py:20-60). Silent on anything else."""
    path = Path(checkpoint_dir)
    shards = sorted(path.glob("*.safetensors"))
    if not shards:
        return
    found = [m for m in (_SHARD_RE.search(s.name) for s in shards) if m]
    if found:
        total = max(int(m.group(2)) for m in found)
        missing = sorted(set(range(1, total + 1)) - {int(m.group(1)) for m in found})
        if missing:
            names = [f"{i:05d}-of-{total:05d}" for i in missing[:4]]
            raise RuntimeError(f"{path}: incomplete checkpoint -- {total - len(missing)} of "
                               f"{total} shards present, missing {names}"
                               f"{' ...' if len(missing) > 4 else ''}")
    index_path = path / "model.safetensors.index.json"
    if index_path.exists():
        weight_map = json.loads(index_path.read_text()).get("weight_map", {})
        absent = sorted(f for f in set(weight_map.values()) if not (path / f).exists())
        if absent:
            raise RuntimeError(f"{path}: the safetensors index references {len(absent)} "
                               f"file(s) that are not present: {absent[:4]}")


class ExpertOffsetIndex:
    """{layer name (the shard's stem): {expert id: {tensor key: ExpertTensorMeta}}}, plus
    the whole-tensor metas of fused layouts in `fused_layer_tensors`."""

    CACHE_VERSION = 2
    CACHE_FILENAME = "vaayu_expert_offsets.json"
    # the routed-expert count's config fields, in order (the top-k and widths that also
    # mention experts are not counts)
    _EXPERT_COUNT_FIELDS = ("num_experts", "num_local_experts", "n_routed_experts")

    def __init__(self, checkpoint_path: str, config_path: str | None = None):
        self.checkpoint_path = Path(checkpoint_path)
        self.config_path = Path(config_path) if config_path is not None else self.checkpoint_path
        self.index: dict = {}
        self.fused_layer_tensors: dict = {}

    @classmethod
    def expert_count_in(cls, config) -> int | None:
        """The routed-expert count a parsed config.json (dict) or config object names."""
        get = config.get if isinstance(config, dict) else (lambda f: getattr(config, f, None))
        for field in cls._EXPERT_COUNT_FIELDS:
            v = get(field)
            if isinstance(v, int) and not isinstance(v, bool) and v > 0:
                return v
        return None

    def expected_expert_count(self) -> int | None:
        """The config's routed-expert count, or None (no config, or not an MoE config)."""
        p = self.config_path / "config.json"
        if not p.exists():
            return None
        try:
            config = json.loads(p.read_text())
        except (OSError, ValueError):
            return None
        return self.expert_count_in(config)

    @staticmethod
    def _fused_expert_axis(key: str, shape: list, expected: int | None) -> bool:
        """`key` holds every expert on its leading axis: under an `experts.` prefix with no
        numeric component, at least 2-D, leading dimension = the config's expert count."""
        if expected is None or len(shape) < 2 or shape[0] != expected:
            return False
        return _FUSED_EXPERTS_RE.search(key) is not None

    def _put(self, layer, expert, key, meta):
        self.index.setdefault(layer, {}).setdefault(expert, {})[key] = meta

    def build(self, write_cache: bool = True) -> None:
        assert_checkpoint_complete(self.checkpoint_path)
        self.index, self.fused_layer_tensors = {}, {}
        expected = self.expected_expert_count()
        for shard in sorted(self.checkpoint_path.glob("*.safetensors")):
            layer = shard.stem
            header, data_start = read_header(shard)
            for key, meta in header.items():
                if key == "__metadata__":
                    continue
                start, end = meta["data_offsets"]
                if self._fused_expert_axis(key, meta["shape"], expected):
                    self._index_fused(layer, key, meta, data_start + start, end - start,
                                      expected)
                    continue
                m = _EXPERT_RE.search(key)
                if m is not None:
                    self._put(layer, int(m.group(1)), key,
                              ExpertTensorMeta(data_start + start, end - start, meta["shape"],
                                               meta["dtype"]))
        self._assert_experts_found()
        if write_cache:
            self._write_cache()

    def _index_fused(self, layer, key, meta, offset, length, experts) -> None:
        """The whole tensor, and one contiguous range per expert (row-major, expert axis
        leading)."""
        self.fused_layer_tensors.setdefault(layer, {})[key] = ExpertTensorMeta(
            offset, length, meta["shape"], meta["dtype"])
        stride, rem = divmod(length, experts)
        if rem:
            raise RuntimeError(f"{self.checkpoint_path}: fused expert tensor {key!r} is "
                               f"{length} bytes, which does not divide evenly by {experts} "
                               f"experts")
        for e in range(experts):
            self._put(layer, e, key, ExpertTensorMeta(offset + e * stride, stride,
                                                      list(meta["shape"][1:]), meta["dtype"]))

    def _assert_experts_found(self) -> None:
        """An MoE config with an empty index would stream no experts and compute wrong
        output silently: raise instead, naming the expert-like keys seen."""
        expected = self.expected_expert_count()
        if expected is None or self.index:
            return
        seen = []
        for shard in sorted(self.checkpoint_path.glob("*.safetensors")):
            seen = [k for k in read_header(shard)[0] if k != "__metadata__" and "expert" in k.lower()]
            if seen:
                break
        raise RuntimeError(f"{self.checkpoint_path}: config implies {expected} routed experts, "
                           f"but the expert offset index found NONE. Expert-like keys "
                           f"present: {seen[:4] if seen else '(none)'}")

    def _write_cache(self) -> None:
        payload = {
            "__vaayu_index_version__": self.CACHE_VERSION,
            "index": {layer: {str(e): {k: _meta_to_raw(m) for k, m in t.items()}
                              for e, t in experts.items()}
                      for layer, experts in self.index.items()},
            "fused_layer_tensors": {layer: {k: _meta_to_raw(m) for k, m in t.items()}
                                    for layer, t in self.fused_layer_tensors.items()},
        }
        (self.checkpoint_path / self.CACHE_FILENAME).write_text(json.dumps(payload))

    def load_cached(self) -> bool:
        """Read the cache when it is newer than every shard. Version 1 (the bare layer map)
        is read too; it has no fused section."""
        cache = self.checkpoint_path / self.CACHE_FILENAME
        shards = list(self.checkpoint_path.glob("*.safetensors"))
        if not cache.exists() or not shards:
            return False
        if cache.stat().st_mtime < max(s.stat().st_mtime for s in shards):
            return False
        raw = json.loads(cache.read_text())
        if raw.get("__vaayu_index_version__") == self.CACHE_VERSION:
            fused, raw = raw.get("fused_layer_tensors", {}), raw["index"]
        else:
            fused = {}
        self.index = {layer: {int(e): {k: _raw_to_meta(v) for k, v in t.items()}
                              for e, t in experts.items()}
                      for layer, experts in raw.items()}
        self.fused_layer_tensors = {layer: {k: _raw_to_meta(v) for k, v in t.items()}
                                    for layer, t in fused.items()}
        return True

    def build_or_load(self) -> None:
        if not self.load_cached():
            print("[Vaayu-MoE] Building expert offset index...")
            self.build()
            n = sum(len(e) for e in self.index.values())
            print(f"[Vaayu-MoE] Expert index built: {n} expert entries across "
                  f"{len(self.index)} MoE layers")
        else:
            print("[Vaayu-MoE] Expert offset index loaded from cache")
            self._assert_experts_found()

    def get_expert_offsets(self, layer_name: str, expert_idx: int):
        return self.index.get(layer_name, {}).get(expert_idx)

    def moe_layer_names(self) -> list:
        return list(self.index.keys())


# ── loading ─────────────────────────────────────────────────────────────────────────────

def _spans(metas: dict) -> list:
    """The tensors' byte ranges merged where they touch: [(start, end, [keys])]."""
    items = sorted(metas.items(), key=lambda kv: kv[1].file_offset)
    spans = []
    for key, m in items:
        a, b = m.file_offset, m.file_offset + m.byte_length
        if spans and a <= spans[-1][1]:
            spans[-1][1] = max(spans[-1][1], b)
            spans[-1][2].append(key)
        else:
            spans.append([a, b, [key]])
    return spans


def _typed(buf: torch.Tensor, meta: ExpertTensorMeta) -> torch.Tensor:
    dtype = SAFETENSORS_DTYPES[meta.dtype]
    t = buf if buf.data_ptr() % dtype.itemsize == 0 else buf.clone()
    return t.view(dtype).reshape(meta.shape)


def load_expert_tensors(index: ExpertOffsetIndex, layer_name: str, expert_idx: int,
                        device="cpu") -> dict:
    """{key: tensor} of one expert, read with one read per run of touching byte ranges
    (through pinned memory and one host-to-device copy when `device` is a GPU)."""
    metas = index.get_expert_offsets(layer_name, expert_idx)
    if metas is None:
        raise KeyError(f"{layer_name}: expert {expert_idx} is not in the index")
    shard = index.checkpoint_path / f"{layer_name}.safetensors"
    spans = _spans(metas)
    total = sum(b - a for a, b, _ in spans)
    on_gpu = torch.device(device).type == "cuda"
    host = torch.empty(total, dtype=torch.uint8, pin_memory=on_gpu)
    at, where = 0, {}
    with open(shard, "rb") as f:
        for a, b, keys in spans:
            f.seek(a)
            f.readinto(memoryview(host[at:at + (b - a)].numpy()))
            for k in keys:
                where[k] = at + metas[k].file_offset - a
            at += b - a
    buf = host.to(device, non_blocking=True) if on_gpu else host
    return {k: _typed(buf[where[k]:where[k] + metas[k].byte_length], metas[k])
            for k in metas}


def load_resident_experts(index: ExpertOffsetIndex, layer_name: str, device) -> dict:
    """{expert id: blob} for every compressed-tensors expert of one layer, built on
    `device` from the checkpoint's bytes (the blobs `ResidentExperts` and the packed-expert
    kernels take). Raises ValueError for an expert whose roles cannot share one blob."""
    from .moe_patch import _group_packed_tensors_by_weight, build_expert_blob

    blobs = {}
    for e in sorted(index.index.get(layer_name, {})):
        raw = load_expert_tensors(index, layer_name, e, device)
        raw = {k: (v.cpu() if k.endswith("weight_shape") else v) for k, v in raw.items()}
        blob = build_expert_blob(_group_packed_tensors_by_weight(raw))
        if blob is None:
            raise ValueError(f"{layer_name}: expert {e} is not a packed compressed-tensors "
                             f"expert the kernels take")
        blobs[e] = blob
    return blobs
