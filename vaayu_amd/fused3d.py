"""Routed fused-3D MXFP4 experts on MI355X: the gpt-oss experts module's two `matmul_ogs`
calls (+ fused SwiGLU) as hand-written HIP grouped GEMMs over the layer's whole expert
tensors, read in place.

The reference delivers a fused-3D layer sparsely (vaayu/routed_fused3d.py:131-238): the
routed experts' rows are copied into persistent `[num_experts, ...]` device buffers and
the model's own experts forward runs over them, i.e. transformers' `Mxfp4GptOssExperts`
calling the vendored `matmul_ogs` twice (gate/up with bias and the gpt-oss SwiGLU fused,
then down with bias and the routing weights) and its finalize sum over each token's slots.
`Fused3DExperts.forward` is that computation over the same buffers and the same routing:

  vaayu_fused3d_gate_up  grouped gate/up GEMM on MFMA, bias + SwiGLU in the epilogue
                         (gate clipped above at `limit`, up to [-limit, limit],
                         s = gate * sigmoid(alpha gate), h = s * (up + 1)), h in bf16
  vaayu_fused3d_down     grouped down GEMM, (acc + bias) * routing weight, rounded to bf16
  vaayu_prefill_reduce   each token's slots summed in ascending expert id, in fp32

Rows are planned as the packed-expert prefill plans them (16-row blocks of one expert,
vaayu/packed_expert_kernels.py:676-717); the tensors' layout is the checkpoint's
(`gate_up_proj_blocks` [E, 2I, H/32, 16] with gate / up rows interleaved, E8M0 scales
[E, 2I, H/32], and the down pair), so nothing is repacked. Without the built library the
forward raises ImportError; there is no CPU substitute.
"""
import torch

from . import _lib
from . import packed_expert_kernels as pk

_BLOCK_M = pk._PF_BLOCK_M
_STEP = 128                      # K codes per step of the kernels' K loop


def _ceil(v: int, m: int) -> int:
    return (v + m - 1) // m * m


class Fused3DExperts:
    """One layer's fused-3D MXFP4 experts. Tensors stay where they are (one device); the
    biases are kept as fp32 copies (the experts module hands them to `matmul_ogs` as
    `.to(torch.float32)`). `alpha` / `limit`: the gpt-oss SwiGLU's (1.702, 7.0 there)."""

    def __init__(self, gate_up_blocks, gate_up_scales, gate_up_bias, down_blocks, down_scales,
                 down_bias, alpha: float = 1.702, limit: float = 7.0):
        E, two_i, hg, sixteen = gate_up_blocks.shape
        if sixteen != 16 or two_i % 2:
            raise ValueError("gate_up blocks must be [E, 2I, H/32, 16]")
        I, H = two_i // 2, hg * 32
        want = {"gate_up_blocks": (gate_up_blocks, (E, 2 * I, H // 32, 16), torch.uint8),
                "gate_up_scales": (gate_up_scales, (E, 2 * I, H // 32), torch.uint8),
                "gate_up_bias": (gate_up_bias, (E, 2 * I), None),
                "down_blocks": (down_blocks, (E, H, I // 32, 16), torch.uint8),
                "down_scales": (down_scales, (E, H, I // 32), torch.uint8),
                "down_bias": (down_bias, (E, H), None)}
        dev = gate_up_blocks.device
        for name, (t, shape, dtype) in want.items():
            if tuple(t.shape) != shape:
                raise ValueError(f"{name} is {tuple(t.shape)}, expected {shape}")
            if dtype is not None and t.dtype != dtype:
                raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
            if not t.is_contiguous():
                raise ValueError(f"{name} must be contiguous")
            if t.device != dev:
                raise ValueError(f"{name} is on {t.device}, not {dev}")
        if I % 32:
            raise ValueError("the intermediate size must be a multiple of 32")
        self.E, self.H, self.I = E, H, I
        self.Hp, self.Ip = _ceil(H, _STEP), _ceil(I, _STEP)
        self.device = dev
        self.alpha, self.limit = float(alpha), float(limit)
        self.gu_codes, self.gu_scales = gate_up_blocks, gate_up_scales
        self.dn_codes, self.dn_scales = down_blocks, down_scales
        self.gu_bias = gate_up_bias.to(torch.float32).contiguous()
        self.dn_bias = down_bias.to(torch.float32).contiguous()
        # per-expert byte strides of each tensor
        self._stride = {"gu_c": 2 * I * H // 2, "gu_s": 2 * I * H // 32, "dn_c": H * I // 2,
                        "dn_s": H * I // 32, "gu_b": 2 * I * 4, "dn_b": H * 4}

    def _end(self, t):
        return t.data_ptr() + t.numel() * t.element_size()

    def tensors(self) -> dict:
        """The six per-expert tensors the kernels read, by constructor argument name."""
        return {"gate_up_blocks": self.gu_codes, "gate_up_scales": self.gu_scales,
                "gate_up_bias": self.gu_bias, "down_blocks": self.dn_codes,
                "down_scales": self.dn_scales, "down_bias": self.dn_bias}

    def like(self, tensors: dict) -> "Fused3DExperts":
        """The same module (alpha, limit) over other tensors of the same geometry."""
        return Fused3DExperts(**tensors, alpha=self.alpha, limit=self.limit)

    def tables(self, expert_ids):
        """The call's device tables from ONE pinned copy: (gate/up table, down table,
        gate/up bias table, down bias table, rows, slot order, n_blocks, work lists)."""
        eidx = expert_ids.to("cpu", torch.int64)
        if eidx.numel() and (int(eidx.min()) < 0 or int(eidx.max()) >= self.E):
            raise ValueError(f"expert ids must be in [0, {self.E})")
        n, top_k = eidx.shape
        order, live, counts = pk._prefill_plan(eidx)
        nblk = (counts + _BLOCK_M - 1) // _BLOCK_M
        n_blocks = int(nblk.sum())
        lay = torch.arange(live.numel(), dtype=torch.int64)      # ascending expert id
        first_blk = torch.empty_like(nblk)
        first_blk[lay] = nblk[lay].cumsum(0) - nblk[lay]
        owner = torch.repeat_interleave(torch.arange(live.numel()), counts)
        first_row = counts.cumsum(0) - counts
        dest = ((first_blk * _BLOCK_M)[owner] + torch.arange(order.numel())
                - first_row[owner])
        rows = torch.full((n_blocks * _BLOCK_M,), -1, dtype=torch.int64)
        rows[dest] = order
        e_blk = torch.repeat_interleave(live[lay], nblk[lay])
        st = self._stride
        cols = [torch.stack([self.gu_codes.data_ptr() + e_blk * st["gu_c"],
                             self.gu_scales.data_ptr() + e_blk * st["gu_s"]], 1).reshape(-1),
                torch.stack([self.dn_codes.data_ptr() + e_blk * st["dn_c"],
                             self.dn_scales.data_ptr() + e_blk * st["dn_s"]], 1).reshape(-1),
                self.gu_bias.data_ptr() + e_blk * st["gu_b"],
                self.dn_bias.data_ptr() + e_blk * st["dn_b"], rows]
        slot_order = (torch.argsort(eidx, dim=1, stable=True)
                      + (torch.arange(n) * top_k)[:, None]).reshape(-1)
        n_cus = pk._cu_count(self.device)
        blk = nblk[lay].tolist()
        w_gu, s_gu, r_gu = pk._prefill_work(blk, pk._run_blocks(0), -(-self.I // 128), n_cus)
        w_dn, s_dn, r_dn = pk._prefill_work(blk, pk._down_run(blk, -(-self.H // 128), n_cus, self.I))
        parts = cols + [slot_order, w_gu, w_dn]
        dev = pk._PF_TABLES.put(torch.cat(parts), self.device)
        out, at = [], 0
        for t in parts:
            out.append(dev[at:at + t.numel()])
            at += t.numel()
        work = pk.PrefillWork(out[-2], s_gu, out[-1], s_dn, r_dn, r_gu)
        return (*out[:-2], n_blocks, work)

    def forward(self, x, expert_ids, routing_weights):
        """x [tokens, H] bf16; expert_ids [tokens, top_k] (any device; read on the host);
        routing_weights [tokens, top_k] on x's device (the `gammas`). Returns [tokens, H]
        bf16: each token's slots summed in ascending expert id."""
        lib = pk._require_backend()
        if x.dtype != torch.bfloat16 or x.dim() != 2 or x.shape[1] != self.H:
            raise ValueError(f"x must be a bf16 [tokens, {self.H}] tensor")
        T, top_k = expert_ids.shape
        if T != x.shape[0] or tuple(routing_weights.shape) != (T, top_k):
            raise ValueError("x, expert_ids and routing_weights disagree on the call's shape")
        out = torch.empty(T, self.H, dtype=torch.float32, device=x.device)
        if T == 0:
            return out.to(x.dtype)
        # the kernels address x and h rows with 32-bit offsets: a larger call runs in token
        # chunks, with the same bits (a row's arithmetic does not depend on its launch-mates)
        step = pk._tokens_per_launch(self.Hp, self.Ip, top_k, self.E)
        for t0 in range(0, T, step):
            part = slice(t0, min(t0 + step, T))
            self._forward_part(x[part], expert_ids[part], routing_weights[part], out[part])
        return out.to(x.dtype)

    def _forward_part(self, x, expert_ids, routing_weights, out) -> None:
        T, top_k = expert_ids.shape
        gu_t, dn_t, gu_b, dn_b, rows, order, n_blocks, work = self.tables(expert_ids)
        if self.Hp == self.H and x.is_contiguous():
            xp = x
        else:
            xp = torch.zeros(T, self.Hp, dtype=x.dtype, device=x.device)
            xp[:, :self.H] = x
        h = (torch.empty if self.Ip == self.I else torch.zeros)(
            T * top_k, self.Ip, dtype=x.dtype, device=x.device)
        y = torch.empty(T * top_k, self.H, dtype=torch.float32, device=x.device)
        gammas = routing_weights.reshape(-1).to(torch.float32).contiguous()
        self.launch(xp, h, y, out, (gu_t, dn_t, gu_b, dn_b, rows, order, n_blocks, work),
                    gammas, top_k)

    def launch(self, xp, h, y, out, tables, gammas, top_k) -> None:
        """The three kernels on prepared buffers (what `forward` runs; allocates nothing, so
        a caller can record it in a graph): xp [tokens, Hp] bf16 with zero padding columns,
        h [tokens * top_k, Ip] bf16 with zero padding columns, y [tokens * top_k, H] fp32,
        out [tokens, H] fp32, `tables` from `tables()`, gammas fp32 [tokens * top_k]."""
        lib = pk._require_backend()
        gu_t, dn_t, gu_b, dn_b, rows, order, n_blocks, work = tables
        st = _lib.stream_ptr(xp.device)
        rc = lib.vaayu_fused3d_gate_up(
            xp.data_ptr(), rows.data_ptr(), gu_t.data_ptr(), gu_b.data_ptr(),
            work.gate_up.data_ptr(), work.gate_up_slots, work.gate_up_run, h.data_ptr(),
            n_blocks, top_k, self.H, self.Hp, self.I, self.Ip, self._end(self.gu_codes),
            self._end(self.gu_scales), self.alpha, self.limit, st)
        _lib.check(rc, "vaayu_fused3d_gate_up")
        rc = lib.vaayu_fused3d_down(
            h.data_ptr(), rows.data_ptr(), dn_t.data_ptr(), dn_b.data_ptr(),
            work.down.data_ptr(), work.down_slots, work.down_run, gammas.data_ptr(),
            y.data_ptr(), n_blocks, top_k, self.H, self.I, self.Ip, self._end(self.dn_codes),
            self._end(self.dn_scales), st)
        _lib.check(rc, "vaayu_fused3d_down")
        pk._reduce(y, order, out, top_k)


# ── load-time check: the kernels read only the routed experts' rows ───────────────────────

def check_routed_reads(experts, top_k: int, seed: int = 0) -> tuple:
    """Show on random inputs that only the routed experts' rows reach the output
    (the contract of vaayu/routed_fused3d.py:241-345). Returns (passed, reason).

    For M = 1 and M = max(2, E // (2 top_k)) tokens with random routing: run `experts`,
    then run a copy of it whose every NON-routed expert row, in all six tensors, holds
    random bytes (NaN / Inf bf16 and fp32 patterns and E8M0 0xFF included, which is what
    an unread row may hold), and require bitwise-equal outputs. Fails closed: a call that
    routes every expert (nothing left to fill), a difference, or any exception gives
    (False, reason). The copy costs one layer's tensors of device memory for the check."""
    E, H, dev = experts.E, experts.H, experts.device
    g = torch.Generator().manual_seed(seed)
    m_multi = max(2, E // (2 * max(1, int(top_k))))
    try:
        for m in (1, m_multi):
            x = torch.randn(m, H, generator=g).to(device=dev, dtype=torch.bfloat16)
            ids = torch.stack([torch.randperm(E, generator=g)[:top_k] for _ in range(m)])
            w = torch.randn(m, top_k, generator=g).softmax(-1).to(dev)
            routed = sorted(set(ids.reshape(-1).tolist()))
            if len(routed) >= E:
                return False, (f"vacuous at M={m}: all {E} experts were routed, so no row "
                               f"was left to fill")
            out_real = experts.forward(x, ids, w)
            keep = torch.tensor(routed, device=dev)
            filled = {}
            for name, t in experts.tensors().items():
                raw = t.contiguous().view(torch.uint8)
                noise = torch.randint(0, 256, tuple(raw.shape), dtype=torch.uint8,
                                      generator=g).to(dev)
                noise[keep] = raw[keep]
                filled[name] = noise.view(t.dtype).reshape(t.shape)
            out_bad = experts.like(filled).forward(x, ids, w)
            if not torch.equal(out_real, out_bad):
                diff = (out_real.float() - out_bad.float()).abs().max().item()
                return False, (f"non-routed expert rows change the output at M={m} "
                               f"(max|diff| {diff:.3e}): the kernels read rows they were "
                               f"not routed to")
        return True, (f"non-routed expert rows do not change the output at M=1 and "
                      f"M={m_multi}")
    except Exception as e:  # noqa: BLE001 -- fails closed; the reason is returned
        return False, f"self-check raised {type(e).__name__}: {e}"


_ROUTED_VERDICTS: dict = {}


def geometry_key(experts, top_k: int) -> tuple:
    return (experts.E, experts.H, experts.I, experts.alpha, experts.limit, int(top_k))


def routed_reads_verdict(experts, top_k: int, name: str = "this layer") -> bool:
    """`check_routed_reads` once per geometry (experts, sizes, SwiGLU constants, top_k),
    with one line printed when it is decided: the kernels are used for a geometry that
    passes; a failing one is a WARNING, and its layers keep the experts module's own
    forward (vaayu/routed_fused3d.py:348-386 decides routed delivery the same way)."""
    key = geometry_key(experts, top_k)
    if key not in _ROUTED_VERDICTS:
        ok, why = check_routed_reads(experts, top_k)
        _ROUTED_VERDICTS[key] = ok
        if ok:
            print(f"[Vaayu-MoE] fused-3D kernels ON for {name}'s geometry ({why}): only "
                  f"the routed experts' rows are read.")
        else:
            print(f"[Vaayu-MoE] WARNING: fused-3D kernels OFF for {name}'s geometry -- "
                  f"{why}. Its layers keep the experts module's own forward.")
    return _ROUTED_VERDICTS[key]
