"""The prefill tables' host layout (vaayu_amd/packed_expert_kernels.py: _prefill_layout,
_prefill_work) on the CPU: every routed row once, each expert's rows in ascending order over
contiguous blocks padded with -1 (the block structure of vaayu/packed_expert_kernels.py:
691-717), and work lists that cover every block once, in runs of one expert, and spread
the kernels' work over the eight XCDs."""
import numpy as np
import torch

import vaayu_amd.packed_expert_kernels as pk


def _zipf(tokens, experts, top_k, seed):
    g = torch.Generator().manual_seed(seed)
    p = 1.0 / (torch.randperm(experts, generator=g).double() + 1.0) ** 1.1
    return torch.multinomial(p.expand(tokens, experts), top_k, replacement=False, generator=g)


def _runs(work):
    """(XCD, first block, length) of each entry of a work list."""
    w = work.reshape(-1, 8)
    return [(x, int(e) >> 5, int(e) & 31) for k in range(w.shape[0]) for x in range(8)
            for e in [w[k, x]] if int(e) >= 0]


def test_every_row_once_in_its_experts_blocks():
    for seed in range(12):
        g = torch.Generator().manual_seed(seed)
        tokens = int(torch.randint(1, 700, (1,), generator=g))
        experts = int(torch.randint(2, 260, (1,), generator=g))
        top_k = min(8, experts)
        eidx = _zipf(tokens, experts, top_k, seed)
        plan = pk._prefill_plan(eidx)
        order, live, counts = plan
        lay, blocks, rows = pk._prefill_layout(plan)
        assert sorted(lay.tolist()) == list(range(live.numel()))
        assert torch.equal(blocks, (counts + 15) // 16)
        assert rows.numel() == int(blocks.sum()) * 16
        real = rows[rows >= 0]
        assert sorted(real.tolist()) == list(range(tokens * top_k))
        flat = eidx.reshape(-1)
        at = 0
        for i in lay.tolist():
            seg = rows[at * 16:(at + int(blocks[i])) * 16]
            n = int(counts[i])
            assert (seg[n:] == -1).all(), "padding at the end of the expert's blocks"
            mine = seg[:n]
            assert (flat[mine] == live[i]).all(), "a block holds only its expert's rows"
            assert (mine[1:] > mine[:-1]).all(), "rows in ascending order"
            at += int(blocks[i])


def test_work_lists_cover_every_block_once_in_runs_of_one_expert():
    for seed in range(8):
        g = torch.Generator().manual_seed(seed)
        blocks = torch.randint(1, 40, (int(torch.randint(1, 300, (1,), generator=g)),),
                               generator=g).tolist()
        starts = np.cumsum([0] + blocks)
        for run in (8, 16):
            work, n_slots, longest = pk._prefill_work(blocks, run)
            assert longest == min(run, max(blocks))
            assert work.dtype == torch.int64 and work.numel() == n_slots * 8
            runs = _runs(work)
            n_runs = sum(-(-b // run) for b in blocks)
            assert len(runs) == n_runs and n_slots == -(-n_runs // 8)
            seen = np.zeros(int(starts[-1]), dtype=int)
            for _x, first, n in runs:
                assert 1 <= n <= run
                e = int(np.searchsorted(starts, first, side="right")) - 1
                assert (first - starts[e]) % run == 0, "runs start R blocks apart"
                assert first + n <= starts[e + 1], "a run stays inside its expert"
                seen[first:first + n] += 1
            assert (seen == 1).all(), "every block in exactly one run"
            assert work.tolist() == pk._prefill_work(list(blocks), run)[0].tolist()


def test_work_lists_spread_the_work_over_the_xcds():
    """DeepSeek-V3 2048-token Zipf routing (top-8 of 256) and other seeds, runs of 8 and 16
    blocks: the busiest XCD holds at most 5 % more work (`_run_cost`) than the mean."""
    for seed in range(6):
        eidx = _zipf(2048, 256, 8, seed)
        _order, live, counts = pk._prefill_plan(eidx)
        blocks = ((counts + 15) // 16).tolist()
        for run in (8, 16):
            load = np.zeros(8)
            for x, _first, n in _runs(pk._prefill_work(blocks, run)[0]):
                load[x] += pk._run_cost(n)
            assert load.max() / load.mean() < 1.05, (seed, run, load)


def test_run_lengths_chosen_per_call():
    """Gate/up: one long expert is cut into runs of 8, so its 2048 rows fill the 256 CUs,
    while a Zipf-routed call keeps runs of 16. Down: the kernel for runs of up to 16 blocks
    only where it halves the runs over a long K (experts of 8-9 blocks, K 14336), not for
    Zipf routing nor a short K."""
    assert pk._run_length([128], 16, 16, 256) == 8
    eidx = _zipf(2048, 256, 8, 0)
    blocks = ((pk._prefill_plan(eidx)[2] + 15) // 16).tolist()
    assert pk._run_length(blocks, 16, 16, 256) == 16
    assert pk._down_run(blocks, 56, 256, 2048) == 8
    mixtral = [9, 9, 8, 9, 8, 8, 9, 8]
    assert pk._down_run(mixtral, 32, 256, 14336) == 9
    assert pk._down_run([16] * 32, 23, 256, 2880) == 8      # gpt-oss-20b: a short K
    assert pk._down_run([1, 2, 1, 3], 16, 256, 14336) <= 3
