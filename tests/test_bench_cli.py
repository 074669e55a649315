"""bench.py on the CPU: the one-GPU contract, the work formulas the roofline
figures divide by, and the optional power telemetry when amd-smi is absent."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import bench  # noqa: E402


@pytest.mark.parametrize("n", [2, 8])
def test_more_than_one_gpu_exits_with_a_message(n, capsys):
    assert bench.main(["--gpus", str(n)]) == 2
    assert "one GPU" in capsys.readouterr().err


def test_prefill_flops_closed_form():
    # c3: 4 * 128 * 32 * S(S+1)/2 with S = 8192 (causal pairs including the diagonal).
    assert bench.prefill_flops(32, 8192) == 4.0 * 128 * 32 * 8192 * 8193 / 2
    # A suffix at query_start p adds p keys to every one of its rows.
    assert bench.prefill_flops(2, 3, 5) == 4.0 * 128 * 2 * (3 * 5 + 6)
    # Brute force over (row, key) pairs on a tiny case.
    pairs = sum(1 for m in range(7) for n in range(4 + m + 1))
    assert bench.prefill_flops(1, 7, 4) == 4.0 * 128 * pairs


def test_decode_bytes_c4():
    # K and V rows of 8 KV heads at 32769 keys, Q in and O out for 64 heads, f16.
    assert bench.decode_bytes(64, 8, 32769) == 2 * 8 * 32769 * 128 * 2 + 2 * 64 * 128 * 2


def test_power_state_without_amd_smi(monkeypatch):
    monkeypatch.setattr(bench, "AMD_SMI", "/nonexistent/amd-smi")
    assert bench._smi_sample() is None
    assert bench.bench_power_state(None, None, None) is None
