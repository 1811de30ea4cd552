"""The harness-compatible runner on the GPU: the 14 product presets pass the
reference harness's accuracy rule against the runner's torch baseline, and
the timing protocol prints the reference's lines.

Presets 1-13 run at their full shapes (one accuracy trial each, no timing).
Preset 14 (32 x 100 000 tokens, d_model 1024) runs at batch 1 and 4096
tokens: at full size its baseline would score 100 000 x 100 000 per head in
query blocks for hours, as the reference harness itself warns.
"""

import pytest
import torch

import transformer_benchmark as tb

pytestmark = pytest.mark.gpu

PRESET_ARGS = [[("--preset", str(i))] for i in range(1, 14)] + [
    [("--preset", "14"), ("--batch-size", "1"), ("--seq-len", "4096")]]


@pytest.mark.timeout(600)
@pytest.mark.parametrize("flags", PRESET_ARGS, ids=[" ".join(v for _, v in f) for f in PRESET_ARGS])
def test_preset_accuracy(kernels, flags, capsys):
    argv = [x for pair in flags for x in pair] + ["--accuracy-trials", "1", "--skip-benchmark"]
    with capsys.disabled():
        print(f"\n[runner] {' '.join(argv)}", flush=True)
    rc = tb.main(argv)
    out = capsys.readouterr().out
    summary = [line for line in out.splitlines() if line.startswith("summary:")]
    with capsys.disabled():
        print(f"[runner] {summary[-1] if summary else out[-400:]}", flush=True)
    assert rc == 0 and summary and summary[-1].startswith("summary: PASS"), out[-2000:]


def test_timing_lines(kernels, capsys):
    rc = tb.main(["--preset", "2", "--accuracy-trials", "2", "--warmup", "3", "--repeats", "10",
                  "--benchmark-rounds", "2"])
    out = capsys.readouterr().out
    assert rc == 0, out[-2000:]
    lines = out.splitlines()
    assert any(line.startswith("summary: PASS") for line in lines)
    base = [line for line in lines if line.startswith("baseline : median=")]
    opt = [line for line in lines if line.startswith("optimized: median=")]
    speed = [line for line in lines if line.startswith("speedup  : ")]
    assert base and opt and speed, out[-2000:]
    assert float(speed[0].split()[2].rstrip("x")) > 0


def test_streamed_slices_and_chunked_baseline(kernels, capsys, monkeypatch):
    """With the memory budget cut to 1/2000 of what is free, a shape runs as
    batch slices and its baseline scores query blocks, and still passes."""
    real = tb.free_budget
    monkeypatch.setattr(tb, "free_budget", lambda dev: real(dev) // 2000)
    rc = tb.main(["--batch-size", "8", "--seq-len", "2048", "--d-model", "256", "--heads", "4",
                  "--ffn-dim", "512", "--layers", "1", "--causal", "--accuracy-trials", "1",
                  "--warmup", "1", "--repeats", "3", "--benchmark-rounds", "1"])
    out = capsys.readouterr().out
    assert rc == 0, out[-2000:]
    assert "streaming:" in out and "queries at a time" in out, out[-2000:]
    assert "summary: PASS" in out
