"""The full-depth BASELINE config-5 decoder on the device (GPU): Qwen2.5-0.5B shapes,
24 layers, hidden 896, 14 / 2 heads, MLP 4864, vocabulary 151936, random weights.

The float64 oracle (oracle/model_ref.py) takes minutes at this size, so its results
come from tests/golden/full_depth_qwen2.json, written by tests/golden/make_full_depth.py
from the same seeded weights; the test re-draws the weights and runs the device
decoder (weights quantized on the device, symmetric int4 or MXFP4, as bench.py's
decoder does) against it.

W4A16 and MXFP4 (every kernel fp32): the prompt's last-position logits at 512 fixed
vocabulary indices within 1e-5 * max |logit| (the model tests' bar), and the greedy
continuation token for token (the replayed decode graph, the argmax on the device;
the oracle's best-to-second logit gap is at least 9e-3 * max |logit| at every step).

W4A8 quantizes every activation row to int8, and fp32 summation order decides the
rounding of any element within fp32 noise of a .5 tie. At this depth the oracle's
prompt forward meets 282 elements within 1e-4 int8 steps of a tie, and the random-
weight network amplifies one code moved by one step into a large logit change
(measured on the oracle: one such flip in layer 13 moves the last logits by 2.5e-2 *
max |logit|, one in layer 0 by 9.8e-2). The device's W4A8 logits therefore follow the
oracle only to that level (3.6e-2 measured), and only the first greedy token (gap
7.3e-2) is decidable; the bar 0.25 still fails a wrong layer, head or cache (random
logits are off by about 1). The tie handling itself is checked exactly where the
oracle can search the flips: tests/test_gpu_model.py, two layers at these widths.
"""
import json
from pathlib import Path

import numpy as np
import pytest

from lowbit_amd import model as DM

pytestmark = pytest.mark.gpu

FIXTURE = Path(__file__).resolve().parent / "golden" / "full_depth_qwen2.json"
BAR = {"w4a16": 1e-5, "mxfp4": 1e-5, "w4a8": 0.25}
DECIDABLE = {"w4a16": 6, "mxfp4": 6, "w4a8": 1}  # leading greedy tokens compared


@pytest.fixture(scope="module")
def full():
    fx = json.loads(FIXTURE.read_text())
    cfg = DM.qwen2_config()
    assert (cfg.num_layers, cfg.vocab_size, cfg.hidden_size) == (24, 151936, 896)
    W = DM.random_weights(cfg, seed=fx["seed"], float32_draws=fx["float32_draws"])
    return cfg, W, fx


@pytest.mark.parametrize("backend", ["w4a8", "mxfp4", "w4a16"])
def test_full_depth_logits_and_greedy_decode(full, backend):
    cfg, W, fx = full
    want = fx["backends"][backend]
    nd = DECIDABLE[backend]
    if backend != "w4a8":
        assert min(want["top_gap_rel"][:nd]) > 100 * BAR[backend]  # decidable far above the bar
    else:
        assert want["top_gap_rel"][0] > 2 * 3.6e-2  # twice the measured tie-driven deviation
    m = DM.Model(cfg, W, backend)
    idx = np.asarray(fx["index"])
    logits = m.forward(fx["prompt"])
    assert logits.shape == (cfg.vocab_size,)
    err = np.abs(logits[idx].astype(np.float64) - np.asarray(want["prompt_logits_at_index"]))
    rel = float(err.max() / want["prompt_logits_max_abs"])
    print(f"[{backend}] prompt logits rel err {rel:.3g} (bar {BAR[backend]})")
    assert np.isfinite(logits).all()
    assert rel < BAR[backend]
    got = m.generate(fx["prompt"], fx["n_new"])
    print(f"[{backend}] greedy {got} oracle {want['tokens']}")
    assert len(got) == fx["n_new"] and all(0 <= t < cfg.vocab_size for t in got)
    assert got[:nd] == want["tokens"][:nd]
