"""Token chunking of large prefill calls (CPU: the arithmetic only).

The grouped kernels address activation rows (one per token, hidden bf16 values) and
intermediate rows (one per table row, inter bf16 values) with 32-bit byte offsets, and the
library refuses a launch whose tables could hold rows past 0xF0000000 bytes
(`rows_out_of_reach` in vaayu_amd/csrc/prefill_kernels.hpp). `_tokens_per_launch` sizes the
chunks `_prefill_launch` splits a call into; here every chunk it allows is checked against
the library's rule, restated, on real plans of random and adversarial routings."""
import numpy as np
import pytest
import torch

import vaayu_amd.packed_expert_kernels as pk

LIMIT = 0xF0000000


def library_refuses(n_blocks, top_k, hidden, inter):
    """`rows_out_of_reach` of the gate/up and down entries, restated."""
    rows = n_blocks * 16
    return (rows + top_k - 1) // top_k * 2 * hidden > LIMIT or rows * 2 * inter > LIMIT


def n_blocks_of(eidx):
    _order, _live, counts = pk._prefill_plan(eidx)
    return int(((counts + 15) // 16).sum())


@pytest.mark.parametrize("hidden,inter,top_k,experts", [
    (7168, 2048, 8, 256), (4096, 14336, 2, 8), (2048, 768, 8, 128), (2880, 2944, 4, 32)])
def test_the_chunk_size_keeps_every_launch_in_range(hidden, inter, top_k, experts):
    step = pk._tokens_per_launch(hidden, inter, top_k, experts)
    # worst case for padding: every expert's rows end one past a whole block, so the
    # tables hold tokens * top_k + 15 * experts rows -- a multiple of 16 at most that
    worst = step * top_k + 15 * experts
    assert not library_refuses(worst // 16, top_k, hidden, inter)
    # and it is not loose by more than the padding allowance: that many more tokens, with
    # no padding at all, are refused
    over = step + -(-15 * experts // top_k) + 1
    assert library_refuses(-(-over * top_k // 16), top_k, hidden, inter)


def test_known_chunk_sizes():
    """DeepSeek-V3 (hidden 7168, inter 2048, top-8 of 256): h rows bound it; Mixtral
    (hidden 4096, inter 14336, top-2 of 8): h rows of 28 KiB."""
    assert pk._tokens_per_launch(7168, 2048, 8, 256) == (LIMIT // 4096 - 15 * 256) // 8
    assert pk._tokens_per_launch(4096, 14336, 2, 8) == (LIMIT // 28672 - 15 * 8) // 2
    assert pk._tokens_per_launch(7168, 2048, 8, 256) == 122400
    assert pk._tokens_per_launch(4096, 14336, 2, 8) == 70157


@pytest.mark.parametrize("seed", range(3))
def test_real_plans_of_a_chunk_pass_the_library_rule(monkeypatch, seed):
    """With the limit lowered so a chunk is a few hundred tokens, random routings of one
    chunk's tokens always pass the library's rule at that limit."""
    global LIMIT
    small = 24 << 20
    monkeypatch.setattr(pk, "_OFFSET_LIMIT", small)
    monkeypatch.setattr(__import__(__name__), "LIMIT", small)
    hidden, inter, top_k, experts = 7168, 2048, 8, 256
    step = pk._tokens_per_launch(hidden, inter, top_k, experts)
    g = torch.Generator().manual_seed(seed)
    for _ in range(5):
        eidx = torch.stack([torch.randperm(experts, generator=g)[:top_k] for _ in range(step)])
        assert not library_refuses(n_blocks_of(eidx), top_k, hidden, inter)
    # every expert gets few rows: the most padding a chunk can carry
    eidx = (torch.arange(step * top_k) % experts).reshape(step, top_k)
    assert not library_refuses(n_blocks_of(eidx), top_k, hidden, inter)


def test_a_call_one_token_over_is_split(monkeypatch):
    """`_prefill_launch` launches ceil(tokens / step) chunks, in token order."""
    monkeypatch.setattr(pk, "_OFFSET_LIMIT", 8 << 20)
    hidden, inter, top_k = 2048, 512, 2
    step = pk._tokens_per_launch(hidden, inter, top_k, 4)
    seen = []
    monkeypatch.setattr(pk, "_prefill_call",
                        lambda x, e, w, b, out, plan: seen.append((x.shape[0], int(x[0, 0]))))
    tokens = 2 * step + 1
    x = torch.arange(tokens, dtype=torch.float32)[:, None].expand(tokens, hidden)
    eidx = torch.arange(tokens * top_k).reshape(tokens, top_k) % 4
    blob = {"geom": (4, 128, (("gate", inter, hidden), ("down", hidden, inter),
                                ("up", inter, hidden))), "flat": {}}
    pk._prefill_launch(x, eidx, torch.ones(tokens, top_k), dict.fromkeys(range(4), blob),
                       torch.empty(tokens, hidden))
    assert seen == [(step, 0), (step, step), (1, 2 * step)]
