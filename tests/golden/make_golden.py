"""Write the committed golden fixtures under tests/golden/.

worked_example.npz — the reference's own worked routing example: 16 tokens,
  top-2 over 8 experts (moe/MoE_detailed_computation_dataflow.md:74-91) and the
  per-expert loads it states (:114-122).  Typed in from the note.
oracle_tiny.npz — oracle outputs of every stage on a tiny seeded layer
  (T=32, H=128, E=4, K=2, I=128) as a regression fixture for the oracle and
  the kernels.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import smoe_oracle as O  # noqa: E402

WORKED = [(0, 3), (1, 5), (0, 6), (2, 4), (0, 2), (3, 7), (1, 4), (5, 6), (2, 7), (0, 3), (1, 5),
          (4, 6), (3, 6), (1, 2), (0, 7), (2, 5)]
WORKED_COUNTS = [5, 4, 5, 4, 3, 4, 4, 3]


def tiny_inputs():
    rng = np.random.default_rng(1234)
    T, H, E, K, I = 32, 128, 4, 2, 128
    x = O.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    logits = rng.standard_normal((T, E)).astype(np.float32)
    w1 = O.f32_to_bf16((rng.standard_normal((E, 2 * I, H)) * 0.02).astype(np.float32))
    w2 = O.f32_to_bf16((rng.standard_normal((E, H, I)) * 0.02).astype(np.float32))
    return dict(x=x, logits=logits, w1=w1, w2=w2, K=np.int32(K))


def weight_quant_inputs():
    rng = np.random.default_rng(99)
    return O.f32_to_bf16((rng.standard_normal((2, 128, 256)) * 0.02).astype(np.float32))


def main():
    np.savez_compressed(os.path.join(HERE, "worked_example.npz"),
                        topk_idx=np.array(WORKED, np.int32), counts=np.array(WORKED_COUNTS, np.int32))
    inp = tiny_inputs()
    w1q, w1s = O.quantize_weight_blockwise(inp["w1"])
    w2q, w2s = O.quantize_weight_blockwise(inp["w2"])
    res = O.moe_forward(inp["x"], inp["logits"], w1q, w1s, w2q, w2s, int(inp["K"]))
    keep = {k: inp[k] for k in ("x", "logits", "K")}
    np.savez_compressed(os.path.join(HERE, "oracle_tiny.npz"), **keep, w1q=w1q, w1s=w1s,
                        w2q=w2q, w2s=w2s, **{k: v for k, v in res.items()})
    wb = weight_quant_inputs()
    wq, ws = O.quantize_weight_blockwise(wb)
    np.savez_compressed(os.path.join(HERE, "weight_quant.npz"), w=wb, wq=wq, ws=ws)
    print("wrote fixtures to", HERE)


if __name__ == "__main__":
    main()
