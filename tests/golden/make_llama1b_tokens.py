"""Write the oracle's greedy stream of the centred-code Llama-1B-shaped model
(tests/golden/llama1b_centered_tokens.json).

The weights are drawn by thintensor_amd.synth.make_dense on the GPU's random number
generator (seed 0, int4 codes q in [-7, 7]), so this runs on a machine with the GPU;
the decode itself is the CPU oracle (oracle.decode_ref.DenseRef) from start token 1
at position 512.  The committed JSON holds data only: the parity test checks its live
oracle stream against it, and bench.py compares the timed stream with it.

Usage: python tests/golden/make_llama1b_tokens.py [output.json]
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

STEPS = 64
SEED = 0
START = 1


def main() -> int:
    import torch

    from oracle.decode_ref import DenseRef
    from thintensor_amd.synth import LLAMA_1B, make_dense

    out = Path(sys.argv[1]) if len(sys.argv) > 1 else Path(__file__).with_name("llama1b_centered_tokens.json")
    s = LLAMA_1B
    w = make_dense(s, device=torch.device("cuda:0"), seed=SEED, centered_codes=True)
    ref = DenseRef(w)
    tokens = ref.generate(START, s.prior_tokens, STEPS)
    out.write_text(json.dumps({"model": "llama-3.2-1b-shaped, int4 g128 codes q in [-7, 7]", "seed": SEED,
                               "start_token": START, "position": s.prior_tokens, "tokens": tokens}) + "\n")
    print(f"{len(tokens)} oracle tokens -> {out}: {tokens}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
