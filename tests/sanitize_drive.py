"""Driver for tests/test_oracle_sanitizers.py, run in a subprocess with the
AddressSanitizer and UBSan runtimes preloaded: every composed entry point
of the oracle library given as argv[1] on a 2-layer Qwen2 and a 2-layer
Qwen3 model, including invalid token ids, a rewind, a clamp, and a
generate / ingest that run into max_ctx."""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

from c2slm_amd import gguf as G  # noqa: E402
from oracle import oracle as O  # noqa: E402


def main(lib_path: str, workdir: str) -> None:
    shapes = (("qwen2", G.ModelShape(n_layers=2, n_vocab=4096)),
              ("qwen3", G.ModelShape(n_layers=2, n_embd=512, n_heads=4, n_kv_heads=2, n_ff=768, n_vocab=4096,
                                     arch="qwen3")))
    for arch, shape in shapes:
        path = os.path.join(workdir, f"{arch}.gguf")
        G.write_synthetic_model(path, shape, seed=3)
        gf = G.GGUFFile(path)
        orc = O.OracleEngine(gf, max_ctx=64, n_threads=2, lib_path=lib_path)
        rng = np.random.default_rng(1)
        for pos, t in enumerate(rng.integers(0, 4096, 6).tolist() + [4096 + 3, -1]):
            orc.forward(int(t), pos)
        orc.set_seq_len(0)
        orc.ingest_from(0, rng.integers(0, 4096, 20).astype(np.int32))
        orc.ingest_from(10, rng.integers(0, 4096, 5).astype(np.int32))    # rewind
        orc.ingest_from(1000, rng.integers(0, 4096, 3).astype(np.int32))  # clamp to SeqLen
        orc.compute_logits()
        toks = orc.generate(60, 4094, 4093, 1.15)                          # stops at max_ctx
        orc.ingest_from(60, rng.integers(0, 4096, 10).astype(np.int32))   # stops at max_ctx
        orc.close()
        print(arch, "ok", len(toks), flush=True)


if __name__ == "__main__":
    main(sys.argv[1], sys.argv[2])
