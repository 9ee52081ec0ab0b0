"""Writes tests/golden/decode_fp16_2layer.json: greedy decode of a 2-layer, full-width
Qwen2-VL text decoder (seeded synthetic fp16 weights, omniserver_amd.synth seed 11) by the
CPU oracle in its fp16-faithful mode.  The reference publishes no vectors for this path,
so this fixture pins the oracle against regressions and lets GPU tests compare against
stored values.  Run: python tests/golden/make_golden.py"""

import json
import os
import sys

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import qwen2_ref as ref  # noqa: E402
from omniserver_amd import synth  # noqa: E402
from tests.helpers import oracle_from_fp16  # noqa: E402

SEED, LAYERS, PROMPT_LEN, STEPS = 11, 2, 24, 4
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "decode_fp16_2layer.json")


def generate():
    shape = synth.DecoderShape()
    w = synth.fp16_decoder(shape, seed=SEED, num_layers=LAYERS)
    orc = oracle_from_fp16(w, shape)
    prompts = [synth.random_ids(PROMPT_LEN, shape.vocab_size, 13, f"sp{i}").tolist()
               for i in range(2)]
    kp = [torch.zeros(3, 64, 2, 128) for _ in range(LAYERS)]
    vp = [torch.zeros(3, 64, 2, 128) for _ in range(LAYERS)]
    lens = torch.zeros(3, dtype=torch.int64)
    emb = torch.cat([w["embed"][torch.tensor(p)].float() for p in prompts], 0)
    pos = torch.arange(PROMPT_LEN).view(1, -1).expand(3, -1).repeat(1, 2)
    lg = orc.prefill(emb, pos, [PROMPT_LEN] * 2, [0, 1], kp, vp, lens)
    steps = []
    for s in range(STEPS + 1):
        top = lg.topk(5, dim=-1)
        steps.append({"tokens": ref.greedy(lg),
                      "margin": ref.top2_margin(lg).tolist(),
                      "top5_ids": top.indices.tolist(), "top5_logits": top.values.tolist()})
        if s < STEPS:
            lg = orc.decode_step(steps[-1]["tokens"], kp, vp, lens)
            lens[:2] += 1
    return {"seed": SEED, "layers": LAYERS, "prompts": prompts, "steps": steps,
            "note": "oracle fp16-faithful mode; step 0 = prefill logits at segment ends"}


if __name__ == "__main__":
    data = generate()
    with open(OUT, "w") as f:
        json.dump(data, f)
    print(f"wrote {OUT}")
