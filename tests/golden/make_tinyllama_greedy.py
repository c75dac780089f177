"""Writes tests/golden/tinyllama_greedy.json: the greedy tokens the reference's chatbot
composition (examples/apps/tinyllama/chatbot.tl:174-222 with sample(temp <= 0)) produces on
the CPU oracle for the synthetic TinyLlama-shape Q4_0 model of tl_amd.llama
(synthetic_weights(seed 1234), 512-token prompt synthetic_prompt(seed 1234)).

The oracle's model path is bit-identical to the tl_cpu op chain (see oracle/tl_llama_oracle.c);
it runs multi-threaded (OpenMP) and takes a few minutes here.
"""
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

import oracle  # noqa: E402
from tl_amd.llama import LlamaConfig, synthetic_prompt, synthetic_weights  # noqa: E402

SEED, PROMPT, STEPS = 1234, 512, 32


def main():
    cfg = LlamaConfig.tinyllama(max_seq=2048)
    t0 = time.time()
    m = oracle.Llama(cfg)
    m.load(synthetic_weights(cfg, SEED))
    prompt = synthetic_prompt(cfg, SEED, PROMPT)
    print(f"loaded in {time.time() - t0:.1f} s", flush=True)
    m.reset()
    logits = m.forward(prompt)
    top = np.argsort(logits)[::-1][:2]
    toks, margins = [], [float(logits[top[0]] - logits[top[1]])]
    nxt = oracle.argmax_last(logits)
    toks.append(nxt)
    for _ in range(STEPS - 1):
        logits = m.forward([nxt])
        top = np.argsort(logits)[::-1][:2]
        margins.append(float(logits[top[0]] - logits[top[1]]))
        nxt = oracle.argmax_last(logits)
        toks.append(nxt)
    print(f"done in {time.time() - t0:.1f} s: {toks}", flush=True)
    out = {"generator": "tests/golden/make_tinyllama_greedy.py", "seed": SEED, "prompt_tokens": PROMPT,
           "prompt_head": [int(t) for t in prompt[:8]], "tokens": [int(t) for t in toks],
           "top2_margins": margins}
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "tinyllama_greedy.json"), "w") as f:
        json.dump(out, f, indent=1)


if __name__ == "__main__":
    main()
