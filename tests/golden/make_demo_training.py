"""Writes demo_training.json: the oracle's run of the reference's default
`mesh-gpt train` (src/bin/mesh-gpt.rs:173-299 with its defaults, 47-61 and
config.rs:305-314): the demo corpus, W32 H4 L2 A4 F6, context 32, seed 7,
batches of 8 windows, 1000 AdamW steps (lr 0.003, weight decay 0.01, betas
0.9/0.999), reporting every 100 steps the mean training loss since the last
report and the loss on the fixed validation windows (seed 101).

The gradients are the f64 tape's (og_loss_and_gradient), cast to f32 for the
f32 AdamW update (og_adam); the losses are the tape's f64 values.  Run from
the repository root: python tests/golden/make_demo_training.py (about 2.5
minutes on one core).
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import oracle_lib as O  # noqa: E402


def demo_tokens():
    with open(os.path.join(HERE, "mesh-gpt-demo.txt"), encoding="utf-8") as f:
        text = f.read()
    chars = sorted(set(text))
    index = {ch: i for i, ch in enumerate(chars)}
    return np.array([index[ch] for ch in text], dtype=np.uint32)


def main():
    tokens = demo_tokens()
    c = O.config(vocab_size=26)
    opt = O.Adam(O.initialize(c, 7), learning_rate=0.003, weight_decay=0.01)
    ex, ey = O.text_batch(tokens, True, 32, 8, 101)
    x0, y0 = O.text_batch(tokens, False, 32, 8, 7)
    reports = [{"step": 0, "train": O.loss_and_gradient(c, opt.value, x0, y0, 32)[0],
                "validation": O.loss_and_gradient(c, opt.value, ex, ey, 32)[0]}]
    total, count = 0.0, 0
    for step in range(1, 1001):
        x, y = O.text_batch(tokens, False, 32, 8, 7 + step)
        loss, grad = O.loss_and_gradient(c, opt.value, x, y, 32)
        total += loss
        count += 1
        opt.step(grad)
        if step % 100 == 0:
            reports.append({"step": step, "train": total / count,
                            "validation": O.loss_and_gradient(c, opt.value, ex, ey, 32)[0]})
            total, count = 0.0, 0
            print(reports[-1], flush=True)
    with open(os.path.join(HERE, "demo_training.json"), "w") as f:
        json.dump({"config": "demo corpus, GptConfig::default(), seed 7, batch 8, 1000 steps, AdamW 0.003/0.01",
                   "reports": reports}, f, indent=1)


if __name__ == "__main__":
    main()
