"""The search command's measurement helpers (include/chimera/search_report.hpp)
and its argument handling, on the CPU. Percentiles are pinned against
numpy's linear interpolation (the rule of cpp/apps/utils.cpp:186-197),
recall@k against a hand-worked case of utils.cpp:265-290."""
import subprocess
import struct

import numpy as np
import pytest

from chimera_amd import PKG_DIR

SIZE_MAX = 2**64 - 1
CLI = PKG_DIR / "chimera_search"


@pytest.mark.parametrize("n", [1, 2, 7, 100, 1001])
def test_percentiles_are_linear_interpolation(chimera_mod, n):
    rng = np.random.default_rng(n)
    v = rng.exponential(3.0, size=n)
    s = sorted(v.tolist())
    for p in (0, 25, 50, 90, 95, 99, 100):
        assert chimera_mod.percentile_ms(s, p) == pytest.approx(float(np.percentile(v, p)), rel=1e-12, abs=1e-12)
    # pct is clamped to [0, 100]
    assert chimera_mod.percentile_ms(s, -5) == s[0]
    assert chimera_mod.percentile_ms(s, 150) == s[-1]
    summ = chimera_mod.summarize_query_latencies_ms(v.tolist())
    assert summ["mean_ms"] == pytest.approx(float(v.mean()), rel=1e-12)
    assert summ["stddev_ms"] == pytest.approx(float(v.std(ddof=0)), rel=1e-9, abs=1e-12)
    assert summ["min_ms"] == v.min() and summ["max_ms"] == v.max()
    for key, p in (("p50_ms", 50), ("p90_ms", 90), ("p95_ms", 95), ("p99_ms", 99)):
        assert summ[key] == pytest.approx(float(np.percentile(v, p)), rel=1e-12, abs=1e-12)


def test_empty_latencies(chimera_mod):
    assert chimera_mod.percentile_ms([], 50) == 0.0
    assert all(v == 0.0 for v in chimera_mod.summarize_query_latencies_ms([]).values())


def test_read_gt_tsv(chimera_mod, tmp_path):
    f = tmp_path / "gt.tsv"
    f.write_text("0\t17\t1\n0\t5\t3\nmalformed line\n2\t9\t2\t0.5\n")
    gt = chimera_mod.read_gt_tsv(3, 4, str(f))
    assert gt == [[17, SIZE_MAX, 5, SIZE_MAX], [SIZE_MAX] * 4, [SIZE_MAX, 9, SIZE_MAX, SIZE_MAX]]
    # a missing file leaves the table unfilled
    assert chimera_mod.read_gt_tsv(2, 3, str(tmp_path / "none.tsv")) == [[SIZE_MAX] * 3] * 2
    for bad in ("0\t1\t5\n", "0\t1\t0\n", "3\t1\t1\n"):
        f.write_text(bad)
        with pytest.raises(RuntimeError):
            chimera_mod.read_gt_tsv(3, 4, str(f))


def test_recall_counts_overlap_of_the_first_k(chimera_mod):
    gt = [[1, 2, 3, 4], [5, 6, SIZE_MAX, SIZE_MAX], [7, 8, 9, 10]]
    got = [[4, 3, 99, 1], [6], [10, 9, 8, 7, 1]]
    # k = 3: query 0: got[:3] = {4, 3, 99} vs {1, 2, 3} -> 1; query 1: {6}
    # vs {5, 6, -} -> 1; query 2: {10, 9, 8} vs {7, 8, 9} -> 2
    assert chimera_mod.compute_recall(gt, got, 3) == pytest.approx(4 / 9)
    assert chimera_mod.compute_recall(gt, got, 4) == pytest.approx((3 + 1 + 4) / 12)
    assert chimera_mod.compute_recall(gt, got, 0) == 0.0
    # only the retrieved queries count (the reference evaluates nq of them)
    assert chimera_mod.compute_recall(gt, got[:1], 4) == pytest.approx(3 / 4)


def _run(*args):
    return subprocess.run([str(CLI), *map(str, args)], capture_output=True, text=True, timeout=60)


def test_search_command_arguments(tmp_path):
    if not CLI.exists():
        pytest.fail("chimera_search is not built")
    r = _run("--help")
    assert r.returncode == 0 and "--query <query_embeddings.bin>" in r.stdout and "Default: 3000" in r.stdout
    assert _run().returncode == 0  # no arguments prints the usage
    for args, msg in [(("--bogus",), "Unknown argument: --bogus"), (("--query",), "Missing value for --query"),
                      (("--query", "q", "--gt", "g"), "Missing required arguments."),
                      (("--query", "q", "--gt", "g", "--index", tmp_path / "none"), "--index must point to")]:
        r = _run(*args)
        assert r.returncode == 1 and msg in r.stderr, (args, r.stderr)
    ix = tmp_path / "ix"
    ix.mkdir()
    r = _run("--query", "q", "--gt", "g", "--index", ix)
    assert r.returncode == 1 and "Missing doclens.bin" in r.stderr
    (ix / "doclens.bin").write_bytes(struct.pack("<ii", 1, 3))
    base = ("--query", tmp_path / "q.bin", "--gt", tmp_path / "gt.tsv", "--index", ix)
    for extra, msg in [(("--k", "0"), "--k must be > 0"), (("--warmup", "-1"), "--warmup must be >= 0"),
                       (("--nprobe", "0"), "--nprobe must be > 0"),
                       (("--k-refine", "10", "--k-full-bit", "20"), "--k-full-bit must not exceed --k-refine"),
                       (("--num-chunks", "0"), "--num-chunks must be > 0")]:
        r = _run(*base, *extra)
        assert r.returncode == 1 and msg in r.stderr, (extra, r.stderr)
    # a ground-truth rank past 1000 stops the command with status 0 before
    # any device work, as the reference's does
    q = np.zeros((2, 32, 128), np.float32)
    (tmp_path / "q.bin").write_bytes(struct.pack("<iii", 2, 32, 128) + q.tobytes())
    (tmp_path / "gt.tsv").write_text("0\t1\t1001\n")
    r = _run(*base)
    assert r.returncode == 0 and "exceeds top_k 1000" in r.stderr and "[SEARCH]" not in r.stdout
    # a query length other than 32 is refused
    (tmp_path / "q.bin").write_bytes(struct.pack("<iii", 2, 16, 128) + q.tobytes()[: 2 * 16 * 128 * 4])
    (tmp_path / "gt.tsv").write_text("0\t1\t1\n")
    r = _run(*base)
    assert r.returncode == 1 and "Query length 16" in r.stderr
