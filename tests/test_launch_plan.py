"""The prefill's host launch planners (sophia_amd/csrc/kda_plan.hpp: plan_scan,
plan_segments) on the CPU, built with g++ under AddressSanitizer and
UndefinedBehaviorSanitizer (tests/plan_harness.cpp): hand-worked plans (the
benchmark batch's measured 4/4/4/2/2/1/1/1 slicing, more sequences than the
host ranks, empty sequences, the 4-bit order packing, the segment plan of one
65,536-token sequence) and the plan invariants over random batches, malformed
offsets included (clamped, never an out-of-range read)."""

from __future__ import annotations

import json
import os
import shutil
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NO_SEGMENTS = 8


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    exe = str(tmp_path_factory.mktemp("plan") / "plan_harness")
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
                    "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-I", ROOT,
                    os.path.join(ROOT, "tests", "plan_harness.cpp"), "-o", exe], check=True)

    def run(lines):
        env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
        out = subprocess.run([exe], input="\n".join(lines) + "\n", capture_output=True, text=True, env=env,
                             timeout=120)
        assert out.returncode == 0, out.stderr[-2000:]
        assert "runtime error" not in out.stderr and "AddressSanitizer" not in out.stderr, out.stderr[-2000:]
        return [json.loads(line) for line in out.stdout.splitlines()]
    return run


def _scan_line(cu, heads=16, cus=256, host=True, total=None):
    total = cu[-1] if total is None else total
    return f"scan {len(cu) - 1} {heads} {cus} {total} {int(host)} " + " ".join(str(int(c)) for c in cu)


def _order(plan, n):
    return [(plan["order_bits"] >> (4 * r)) & 15 for r in range(n)]


def _check_scan_invariants(plan, chunks, heads, host):
    n = len(chunks)
    n_cls = plan["n_cls"]
    rank, block, splits = plan["rank"], plan["block"], plan["splits"]
    assert rank[0] == 0 and rank[n_cls] == n and block[0] == 0 and block[n_cls] == plan["blocks"]
    for c in range(n_cls):
        assert rank[c] <= rank[c + 1]
        assert splits[c] in (1, 2, 4, 8)
        pairs = (rank[c + 1] - rank[c]) * heads
        assert block[c + 1] - block[c] == (pairs + 7) // 8 * 8 * splits[c]
        if c:
            assert splits[c] < splits[c - 1]
    if host and n <= 16:
        order = _order(plan, n)
        assert sorted(order) == list(range(n))
        got = [chunks[s] for s in order]
        assert got == sorted(chunks, reverse=True)
        for r in range(n - 1):   # stable: equal chunk counts keep packing order
            if got[r] == got[r + 1]:
                assert order[r] < order[r + 1]
        for r in range(n, 16):
            assert (plan["order_bits"] >> (4 * r)) & 15 == r


def test_benchmark_batch_plan(harness):
    """8 sequences of U[256, 4096] tokens (seed 0) on 256 CUs: longest first,
    4/4/4/2/2/1/1/1 slices, 304 work-groups."""
    lens = [3523, 2702, 2219, 1292, 1438, 413, 544, 319]
    cu = [0] + np.cumsum(lens).tolist()
    plan = harness([_scan_line(cu)])[0]
    assert _order(plan, 8) == [0, 1, 2, 4, 3, 6, 5, 7]
    assert plan["n_cls"] == 3 and plan["splits"][:3] == [4, 2, 1]
    assert plan["rank"][:4] == [0, 3, 5, 8] and plan["block"][:4] == [0, 192, 256, 304]
    _check_scan_invariants(plan, [(n + 63) // 64 for n in lens], 16, True)


def test_more_sequences_than_ranked_and_no_host_copy(harness):
    """Past 16 sequences, or without the host offsets, one class in packing
    order with as many slices as keep every work-group resident."""
    lens = [100 * (i % 7 + 1) for i in range(20)]
    cu = [0] + np.cumsum(lens).tolist()
    many, none = harness([_scan_line(cu), _scan_line(cu[:9], host=False)])
    assert many["n_cls"] == 1 and many["splits"][0] == 1 and many["blocks"] == 20 * 16
    assert _order(many, 16) == list(range(16))
    # 128 pairs: two slices each keep all 256 work-groups resident on 256 CUs
    assert none["n_cls"] == 1 and none["splits"][0] == 2 and none["blocks"] == 8 * 16 * 2
    small = harness([_scan_line([0, 700, 1400], heads=4, host=False)])[0]
    assert small["splits"][0] == 8 and small["blocks"] == 8 * 8   # 8 pairs padded to 8, 8 slices


def test_empty_sequences_and_order_packing(harness):
    """16 sequences in increasing length with three empty ones: the order
    fields hold the reverse packing order, equal chunk counts (1 token and 64
    tokens are one chunk each) and the empty sequences keep packing order, and
    a one-token sequence still gets a slice."""
    lens = [0, 1, 0, 64, 65, 0] + [192 * i for i in range(1, 11)]   # 3 i chunks
    cu = [0] + np.cumsum(lens).tolist()
    plan = harness([_scan_line(cu, heads=2)])[0]
    order = _order(plan, 16)
    assert order[:10] == list(range(15, 5, -1))
    assert order[10:] == [4, 1, 3, 0, 2, 5]   # 2 chunks, 1, 1, then the empty ones
    _check_scan_invariants(plan, [(n + 63) // 64 for n in lens], 2, True)


def test_random_batches_and_malformed_offsets(harness):
    rng = np.random.default_rng(5)
    lines, cases = [], []
    for i in range(300):
        n = int(rng.integers(1, 24))
        heads = int(rng.choice([1, 2, 16, 32]))
        lens = rng.integers(0, 5000, size=n)
        lens[rng.random(n) < 0.2] = 0
        cu = [0] + np.cumsum(lens).tolist()
        total = cu[-1]
        if i % 5 == 4:   # malformed: decreasing, negative and past-the-end offsets
            cu = [int(c) for c in cu]
            j = int(rng.integers(1, n + 1))
            cu[j] = int(rng.choice([-7, total + 999, cu[j] // 3]))
        lines.append(_scan_line(cu, heads=heads, cus=int(rng.choice([64, 256, 304])), total=total))
        chunks = []
        for s in range(n):   # each sequence's pair clamped, as the kernels clamp it
            a = min(max(int(cu[s]), 0), total)
            b = min(max(int(cu[s + 1]), a), total)
            chunks.append((b - a + 63) // 64)
        cases.append((chunks, heads))
    for plan, (chunks, heads) in zip(harness(lines), cases):
        _check_scan_invariants(plan, chunks, heads, True)


def test_segment_plans(harness):
    """One 65,536-token sequence (1,024 chunks): 16 segments of 64 chunks, 15
    composed; two sequences where one is long; off for 5 sequences, for the
    switch, for batches that fill the chip, and for short sequences."""
    lines = [
        "seg 1 16 256 65536 0 0 65536",
        "seg 2 16 256 20000 0 0 9000 20000",
        "seg 5 4 256 90000 0 0 20000 40000 60000 80000 90000",
        f"seg 1 16 256 65536 {NO_SEGMENTS} 0 65536",
        "seg 4 32 256 90000 0 0 20000 40000 60000 90000",
        "seg 2 16 256 9000 0 0 4000 9000",
        "seg 1 16 256 65536 0 0 99999",   # offsets past the end are clamped
    ]
    one, two, five, off, full, short, clamped = harness(lines)
    assert one["on"] and one["run"][:2] == [0, 16] and one["cmp"][:2] == [0, 15]
    assert one["run"][4] == 16 and one["max_segments"] >= 16 and one["run_splits"] == 1
    assert clamped == one
    # 9,000 tokens = 141 chunks -> 3 segments; 11,000 tokens = 172 chunks -> 3
    assert two["on"] and two["run"][:3] == [0, 3, 6] and two["cmp"][:3] == [0, 2, 4]
    for plan in (five, off, full, short):
        assert not plan["on"]
