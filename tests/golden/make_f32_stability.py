"""Writes tests/golden/f32_stability.json: the inputs of the reference's
float64 library calls (softmax exp, the RoPE table's pow/cos/sin) whose
float32 result two float64 libraries of the stated accuracy may round
differently (tests/golden/f32_stability.c).  tests/test_f32_stability.py
recomputes and compares."""
from __future__ import annotations

import json
import os
import re
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "f32_stability.c")
OUT = os.path.join(HERE, "f32_stability.json")
# (max positions, head_dim, theta): the device table's largest max_ctx at the
# Qwen2.5 head_dim and the Qwen3 head_dim
ROPE_CASES = [(36864, 64, 1000000.0), (36864, 128, 1000000.0)]


def run(args) -> str:
    with tempfile.TemporaryDirectory() as td:
        exe = os.path.join(td, "f32_stability")
        subprocess.run(["gcc", "-O2", "-fopenmp", "-o", exe, SRC, "-lm"], check=True)
        return subprocess.run([exe, *args], check=True, capture_output=True, text=True).stdout


def compute() -> dict:
    out = {}
    txt = run(["exp"])
    m = re.search(r"exp inputs (\d+) exceptions (\d+) last_t=(0x[0-9a-f]+)", txt)
    out["exp"] = {"inputs": int(m.group(1)), "last_t": m.group(3),
                  "exceptions": sorted(re.findall(r"^exp t=(0x[0-9a-f]+)", txt, re.M))}
    assert len(out["exp"]["exceptions"]) == int(m.group(2))
    out["rope"] = []
    for P, hd, theta in ROPE_CASES:
        txt = run(["rope", str(P), str(hd), repr(theta)])
        m = re.search(r"rope entries (\d+) exceptions_k1 (\d+) exceptions_k4 (\d+) first_p_k1 (\d+) first_p_k4 (\d+)",
                      txt)
        k1 = sorted((int(a), int(b), c) for a, b, c in re.findall(r"^rope k1 p=(\d+) i=(\d+) (cos|sin)", txt, re.M))
        assert len(k1) == int(m.group(2))
        out["rope"].append({"positions": P, "head_dim": hd, "theta": theta, "entries": int(m.group(1)),
                            "exceptions_k1": int(m.group(2)), "exceptions_k4": int(m.group(3)),
                            "first_position_k1": int(m.group(4)), "first_position_k4": int(m.group(5)),
                            "list_k1": [list(e) for e in k1]})
    return out


if __name__ == "__main__":
    with open(OUT, "w") as f:
        json.dump(compute(), f, indent=1)
    print("wrote", OUT)
