"""Golden teacher-forced decode of BASELINE config 5 at its own positions, from the
float64 oracle (oracle/model_ref.py), for tests/test_gpu_config5_decode.py.

Config 5 is the Qwen2.5-0.5B-shaped decoder (24 layers, hidden 896, 14 / 2 heads,
MLP 4864, vocabulary 151936) with random weights, a 64-token prompt and greedy
decoding; bench.py times it with random_weights(seed=0, float32 draws) and the
prompt default_rng(0).integers(0, 151936, 64), and this fixture uses exactly those.

Per backend (W4A8 and MXFP4, the formats config 5 names, and W4A16; int4 symmetric
as the device model quantizes): the oracle prefills the prompt (logits at all 64
positions) and then decodes N_NEW greedy tokens one at a time through its cache.
For each of the 64 + N_NEW - 1 positions whose next token is predicted it records
the argmax, the gap between the best and second-best logit relative to that row's
max |logit|, the row's max |logit|, the two best tokens and their logits, and the
float64 logits at N_IDX fixed vocabulary indices (arrays in an .npz, keys
`<backend>_<field>`). The device test feeds the same tokens (teacher forcing: the
oracle's greedy tokens, not its own) and compares position by position.

Run from the repository root (about 10 minutes on 8 CPUs):
    python tests/golden/make_config5_decode.py
"""
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from lowbit_amd import formats as F  # noqa: E402
from lowbit_amd import model as DM  # noqa: E402
from oracle import model_ref as MR  # noqa: E402

SEED = 0
PROMPT_LEN = 64
N_NEW = 17          # 16 decode steps after the prefill's token
N_IDX = 128
OUT = Path(__file__).resolve().parent / "config5_decode.npz"


def row_facts(logit: np.ndarray, idx: np.ndarray) -> dict:
    order = np.argsort(logit)[-2:][::-1]  # best, second best
    mx = float(np.abs(logit).max())
    return {"argmax": int(order[0]), "gap_rel": float((logit[order[0]] - logit[order[1]]) / mx), "max_abs": mx,
            "at_index": logit[idx].astype(np.float64), "top2_index": order.astype(np.int64),
            "top2_value": logit[order].astype(np.float64)}


def main() -> None:
    cfg = DM.qwen2_config()
    t0 = time.time()
    W = DM.random_weights(cfg, seed=SEED, float32_draws=True)
    prompt = np.random.default_rng(0).integers(0, cfg.vocab_size, PROMPT_LEN).tolist()
    print(f"weights {time.time() - t0:.1f} s", flush=True)
    idx = np.sort(np.random.default_rng(SEED + 7).choice(cfg.vocab_size, N_IDX, replace=False))
    out = {"seed": np.int64(SEED), "prompt": np.asarray(prompt, np.int64), "n_new": np.int64(N_NEW),
           "index": idx.astype(np.int64)}
    for backend in ("w4a8", "mxfp4", "w4a16"):
        t0 = time.time()
        quant = F.quantize_mxfp4 if backend == "mxfp4" else F.quantize_int4
        ref = MR.RefModel(cfg, W, backend, quant)
        cache = ref.new_cache(PROMPT_LEN + N_NEW)
        rows = [row_facts(r, idx) for r in ref.forward(prompt, cache, logits="all")]
        tokens = [rows[-1]["argmax"]]
        for i in range(N_NEW - 1):
            rows.append(row_facts(ref.forward([tokens[-1]], cache, logits="last"), idx))
            tokens.append(rows[-1]["argmax"])
            print(f"  {backend} step {i + 1}: token {tokens[-1]} gap {rows[-1]['gap_rel']:.3e} "
                  f"({time.time() - t0:.0f} s)", flush=True)
        out[f"{backend}_tokens"] = np.asarray(tokens, np.int64)
        for key in ("argmax", "gap_rel", "max_abs", "at_index", "top2_index", "top2_value"):
            out[f"{backend}_{key}"] = np.asarray([r[key] for r in rows])
        gaps = out[f"{backend}_gap_rel"]
        print(f"{backend}: tokens {tokens}; gaps min {gaps.min():.2e} median {np.median(gaps):.2e} "
              f"({time.time() - t0:.0f} s)", flush=True)
    np.savez_compressed(OUT, **out)
    print("wrote", OUT, OUT.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
