"""Golden decode of the full-depth BASELINE config-5 decoder (Qwen2.5-0.5B shapes:
24 layers, hidden 896, 14 / 2 heads, MLP 4864, vocabulary 151936, tied embeddings)
from the float64 oracle (oracle/model_ref.py), for tests/test_gpu_full_depth.py.

The oracle takes minutes at this size on the CPU (W4A8 re-unpacks its int4 weights
in every call), too long for a GPU test run, so its results are computed once here
and kept as a small JSON fixture; the test re-draws the same random weights from the
seed (numpy's PCG64 float32 normals, the same on every machine) and runs the device
decoder against the fixture.

Per backend (W4A16, MXFP4, W4A8; int4 symmetric as the device model quantizes):
  * the logits of the prompt's last position at 512 fixed vocabulary indices, with
    their float64 max |logit| over the whole vocabulary;
  * the greedy continuation (n_new tokens) and, per step, the oracle's gap between
    its best and second-best logit relative to max |logit| (a step whose gap is
    below the device's error could legitimately decode differently).

Run from the repository root:  python tests/golden/make_full_depth.py
"""
import json
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from lowbit_amd import formats as F  # noqa: E402
from lowbit_amd import model as DM  # noqa: E402
from oracle import model_ref as MR  # noqa: E402

SEED = 21
PROMPT = [5, 17, 33, 2, 90, 1000, 151000, 7]
N_NEW = 6
N_IDX = 512
OUT = Path(__file__).resolve().parent / "full_depth_qwen2.json"


def main() -> None:
    cfg = DM.qwen2_config()
    t0 = time.time()
    W = DM.random_weights(cfg, seed=SEED, float32_draws=True)
    print(f"weights {time.time() - t0:.1f} s", flush=True)
    idx = np.sort(np.random.default_rng(SEED + 1).choice(cfg.vocab_size, N_IDX, replace=False))
    out = {"seed": SEED, "float32_draws": True, "prompt": PROMPT, "n_new": N_NEW, "config": "qwen2_config()",
           "index": idx.tolist(), "backends": {}}
    for backend in ("w4a16", "mxfp4", "w4a8"):
        t0 = time.time()
        quant = F.quantize_mxfp4 if backend == "mxfp4" else F.quantize_int4
        ref = MR.RefModel(cfg, W, backend, quant)
        cache = ref.new_cache(len(PROMPT) + N_NEW)
        logit = ref.forward(PROMPT, cache)
        first = logit
        toks, gaps = [], []
        for i in range(N_NEW):
            top2 = np.sort(logit)[-2:]
            gaps.append(float((top2[1] - top2[0]) / np.abs(logit).max()))
            toks.append(int(np.argmax(logit)))
            if i + 1 < N_NEW:
                logit = ref.forward([toks[-1]], cache)
        out["backends"][backend] = {"tokens": toks, "top_gap_rel": gaps,
                                    "prompt_logits_max_abs": float(np.abs(first).max()),
                                    "prompt_logits_at_index": [float(v) for v in first[idx]]}
        print(f"{backend}: {toks} gaps {[f'{g:.2e}' for g in gaps]} ({time.time() - t0:.0f} s)", flush=True)
    OUT.write_text(json.dumps(out, indent=1))
    print("wrote", OUT)


if __name__ == "__main__":
    main()
