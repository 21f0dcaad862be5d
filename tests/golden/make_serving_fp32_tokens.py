"""Expected FP32 greedy tokens of the requests of the Qwen2.5-0.5B-shape
serving workload (workloads.qwen05b_serving), from the oracle on the CPU.

    python tests/golden/make_serving_fp32_tokens.py

writes tests/golden/serving_qwen05b_fp32_tokens.json: per request (all 48
initial requests and the first eight arrivals) its
id, prompt length, the oracle's greedy tokens for all max_new_tokens, and per
step the top-2 logit margin and the second-best token. At each near tie
(margin below NEAR_TIE) it also stores the branch: the oracle's greedy tokens
had the second-best token been taken there (that token, then greedy decoding
of the rest), with the branch's own margins, so a run that takes the other
side of a near tie is still compared token for token. The model is the
seeded random init of workloads.build_serving (torch.manual_seed(0) before
construction, FP32 on the CPU), so the GPU test rebuilds the same weights.
"""

from __future__ import annotations

import json
import os
import sys
import time

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [REPO, os.path.join(REPO, "mini-llm-runtime_amd")]

from mini_llm_runtime_amd import workloads  # noqa: E402
from mini_llm_runtime_amd.model.qwen2 import TinyQwen2Config, TinyQwen2ForCausalLM  # noqa: E402
from oracle.qwen2_model import OracleQwen2  # noqa: E402

# Every initial request and the first eight arrivals (all of them are
# admitted during the warm-up or early in the measured steps).
SAMPLED = [f"init{i}" for i in range(48)] + [f"arr{i}" for i in range(8)]
OUT = os.path.join(HERE, "serving_qwen05b_fp32_tokens.json")
NEAR_TIE = 1e-3  # must equal tests/test_gpu_runtime.py's NEAR_TIE


def branches(oracle, prompt, tokens, margins, second):
    """The greedy continuation after taking the second-best token at every
    near-tie step of `tokens`."""
    out = []
    for i, m in enumerate(margins):
        if m >= NEAR_TIE:
            continue
        prefix = list(prompt) + tokens[:i] + [second[i]]
        rest = len(tokens) - i - 1
        b_margins: list = []
        cont = oracle.cached_greedy(prefix, rest, b_margins) if rest > 0 else []
        out.append({"step": i, "tokens": [second[i]] + cont,
                    "margins": [m] + [mm for mm, _ in b_margins],
                    "second": [tokens[i]] + [ss for _, ss in b_margins]})
    return out


def main() -> None:
    torch.set_num_threads(os.cpu_count() or 1)
    w = workloads.qwen05b_serving()
    cfg = TinyQwen2Config(**w.config)
    torch.manual_seed(w.model_seed)
    model = TinyQwen2ForCausalLM(cfg).float()
    oracle = OracleQwen2(model.state_dict(), cfg)
    del model
    prompts = {f"init{i}": pm for i, pm in enumerate(w.initial)}
    prompts.update({f"arr{i}": pm for i, pm in enumerate(w.arrivals)})
    out = []
    with torch.no_grad():
        for rid in SAMPLED:
            prompt, max_new = prompts[rid]
            t0 = time.time()
            margins: list = []
            tokens = oracle.cached_greedy(prompt, max_new, margins)
            entry = {"request_id": rid, "prompt_len": len(prompt), "tokens": tokens,
                     "margins": [m for m, _ in margins],
                     "second": [s for _, s in margins]}
            entry["branches"] = branches(oracle, prompt, tokens, entry["margins"],
                                         entry["second"])
            out.append(entry)
            print(f"{rid}: {len(prompt)} prompt tokens, {max_new} new, "
                  f"min margin {min(m for m, _ in margins):.3g}, {time.time() - t0:.1f}s",
                  flush=True)
    with open(OUT, "w") as f:
        json.dump({"workload": w.name, "dtype": "float32", "requests": out}, f)
    print("wrote", OUT)


if __name__ == "__main__":
    main()
