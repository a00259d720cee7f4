"""The kvx_bench command line (kvx_amd/csrc/kvx_bench.cpp) keeps the
reference binary's contract (benchmarks/kvx_bench.cu; checked by the
reference's benchmarks/tests/kvx_bench_cli_test.py:6-49): the flags are
echoed in the "write," CSV row (13 fields, field 12 = tokens_per_seq),
invalid arguments exit non-zero before any GPU work, and the gather row
follows the same header.
"""
import subprocess

import pytest

from conftest import REPO

BIN = REPO / "kvx_amd" / "kvx_bench"
HEADER = ("kernel,seq_count,seq_len,block_size,num_heads,head_dim,num_blocks,iters,warmup,"
          "ms_per,tokens_per_s,gb_per_s,tokens_per_seq")


def run(*args):
    if not BIN.exists():
        pytest.fail(f"{BIN} is not built (python -m kvx_amd.build)")
    return subprocess.run([str(BIN), *args], text=True, capture_output=True, timeout=120)


@pytest.mark.parametrize("args,msg", [
    (["--seq-count", "0"], "Invalid config values."),
    (["--iters=0"], "Invalid config values."),
    (["--head-dim", "-4"], "Invalid config values."),
    (["--seq-len", "4", "--tokens-per-seq", "8"], "tokens_per_seq cannot exceed seq_len."),
    (["--dtype=float64"], "Unsupported --dtype=float64"),
])
def test_invalid_arguments_exit_nonzero(args, msg):
    proc = run(*args)
    assert proc.returncode != 0
    assert msg in proc.stderr
    assert "write," not in proc.stdout


@pytest.mark.gpu
def test_reference_cli_contract():
    proc = run("--seq-count", "2", "--seq-len", "8", "--tokens-per-seq", "2", "--block-size",
               "4", "--num-heads", "2", "--head-dim", "4", "--iters", "1", "--warmup", "1",
               "--dtype=float32")
    assert proc.returncode == 0, proc.stderr
    lines = proc.stdout.splitlines()
    assert HEADER in lines
    write = next(l for l in lines if l.startswith("write,")).split(",")
    gather = next(l for l in lines if l.startswith("gather,")).split(",")
    assert len(write) == 13 and len(gather) == 13
    assert (int(write[1]), int(write[2]), int(write[3]), int(write[12])) == (2, 8, 4, 2)
    assert (int(write[4]), int(write[5]), int(write[6])) == (2, 4, 4)  # heads, dim, blocks
    assert float(write[9]) > 0 and float(gather[9]) > 0


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_decode_and_separate_value_flags(dtype):
    proc = run("--seq-count=4", "--seq-len=100", "--block-size=16", "--num-heads=8",
               "--head-dim=128", "--iters=3", "--warmup=1", "--dtype", dtype)
    assert proc.returncode == 0, proc.stderr
    gather = next(l for l in proc.stdout.splitlines() if l.startswith("gather,")).split(",")
    assert (int(gather[1]), int(gather[2]), int(gather[6]), int(gather[12])) == (4, 100, 28, 1)
