"""Writes tests/golden/tiny_greedy.json: the oracle's teacher-forced pass
over a seeded 32-token prompt followed by 16 greedy tokens on the tiny
qwen4_exp configuration (presets.tiny(), seed 1234, q8 KV).  Per position:
the greedy token (lowest index on ties), its margin over the runner-up,
the top-5 ids, and a digest of the logits (sum, sum of squares, first 8).

The reference ships no numeric vectors for model outputs (its end-to-end
known answer needs checkpoint weights that are not in the repository), so
these fixtures pin regressions of the oracle and of the HIP engine against
one another.  Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

PROMPT_SEED, PROMPT_LEN, GEN = 32, 32, 16
OUT = Path(__file__).with_name("tiny_greedy.json")


def digest(logits: np.ndarray) -> dict:
    order = np.argsort(-logits.astype(np.float64), kind="stable")
    top = order[:5]
    return {
        "argmax": int(order[0]),
        "margin": float(logits[order[0]] - logits[order[1]]),
        "top5": [int(i) for i in top],
        "sum": float(np.sum(logits, dtype=np.float64)),
        "sumsq": float(np.sum(logits.astype(np.float64) ** 2)),
        "head": [float(v) for v in logits[:8]],
    }


def generate() -> dict:
    from cherenkov_amd import presets
    from oracle.oracle import OracleModel

    cfg = presets.tiny()
    prompt = np.random.default_rng(PROMPT_SEED).integers(0, cfg.vocab_size, PROMPT_LEN).tolist()
    st = OracleModel(cfg).new_state()
    steps = []
    tok = None
    for i in range(PROMPT_LEN + GEN):
        inp = prompt[i] if i < PROMPT_LEN else tok
        d = digest(st.forward_token(inp, True))
        d["input"] = int(inp)
        steps.append(d)
        tok = d["argmax"]
    return {"config": "presets.tiny(seed=1234)", "kv": "q8", "prompt": prompt, "steps": steps}


if __name__ == "__main__":
    OUT.write_text(json.dumps(generate(), indent=1) + "\n")
    print(f"wrote {OUT}")
