"""Writes tests/golden/model_*.npz: logits of the reference's own
mia_model_step (src/model/forward.c:199-217, through oracle/_ref built from
the reference sources: mia_file.c, expert_cache.c, forward.c, quant.c,
matmul.c) on synthetic .mia files written by tests/mia_writer.py.

Run in the container that holds the reference sources, after
`make -C oracle ref`:

    python tests/golden/make_golden_model.py

Each fixture holds the model's shape and seed, the SHA-256 of the .mia file
the writer produces from them, the tokens (positions 0..n-1) and the
reference's logits as raw bits.
"""
import hashlib
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

import oracle as O  # noqa: E402
import mia_writer as MW  # noqa: E402

# tools/e2e/e2e_test.go:21 (the reference's e2e token list)
E2E_TOKENS = [1, 5, 9, 33, 2, 77, 64, 5, 5, 90, 12, 0]
MODELS = {
    "model_tiny": dict(cfg=MW.TINY, seed=7, tokens=E2E_TOKENS, max_seq=16, slots=2),
    "model_mini_qwen": dict(cfg=MW.MINI_QWEN, seed=9, tokens=[3, 17, 42, 5], max_seq=8, slots=4),
}


def main():
    manifest = {}
    for name, spec in MODELS.items():
        with tempfile.TemporaryDirectory() as tmp:
            path = os.path.join(tmp, name + ".mia")
            MW.synthetic(O, path, spec["cfg"], MW.Q8_0, spec["seed"])
            digest = hashlib.sha256(open(path, "rb").read()).hexdigest()
            logits = O.ref_model_logits(path, spec["tokens"], spec["max_seq"], spec["slots"])
        np.savez(os.path.join(HERE, name + ".npz"), tokens=np.array(spec["tokens"], np.int32),
                 logits_bits=logits.view(np.uint32), file_sha256=np.array(digest),
                 seed=np.array(spec["seed"]), max_seq=np.array(spec["max_seq"]))
        manifest[name] = dict(cfg=spec["cfg"], seed=spec["seed"], tokens=spec["tokens"],
                              max_seq=spec["max_seq"], cache_slots=spec["slots"],
                              file_sha256=digest)
        print(name, logits.shape, digest[:16])
    json.dump(manifest, open(os.path.join(HERE, "MANIFEST_model.json"), "w"), indent=1)


if __name__ == "__main__":
    main()
