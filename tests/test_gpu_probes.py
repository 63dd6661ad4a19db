"""The measurement probes on the GPU: the hand-off litmus across XCDs (the layer's
rules lose no word: write-once data read plain after its counter, and a line polled
while partly published read device-coherently) and the streaming-read probe."""

import sys

import pytest
import torch

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return "cuda:0"


@pytest.mark.parametrize("mode", [0, 1, 3])
def test_handoff_rules_lose_no_word(mode):
    from sgl_amd_mono.k2 import probes
    dev = _dev()
    print(f"handoff litmus mode {mode}", flush=True)
    bad, gave_up, us = probes.handoff(mode, rounds=50, dev=dev)
    assert gave_up == 0, f"mode {mode}: {gave_up} bounded waits gave up"
    assert bad == 0, f"mode {mode}: {bad} stale words"


def test_handoff_partial_line_plain_read_runs():
    # the form the layer avoids: reported, not asserted (stale words are possible)
    from sgl_amd_mono.k2 import probes
    dev = _dev()
    bad, gave_up, us = probes.handoff(2, rounds=50, dev=dev)
    print(f"partly published line, plain read: {bad} stale words, {us:.2f} us a round", file=sys.stderr)
    assert gave_up == 0


def test_stream_read_probe():
    from sgl_amd_mono.k2 import probes
    dev = _dev()
    nbytes, b2b, cold = probes.stream_read(64, reps=3, launches=8, dev=dev)
    assert nbytes >= 64 << 20
    assert 500 < max(b2b) < 8000 and 100 < max(cold) < 8000, (b2b, cold)
