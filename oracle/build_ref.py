"""Compile the reference's own in-test C dequantisation oracles into oracle/_ref/.

The reference keeps three C99 oracles as string constants inside its Go test
files (tensor/oracle_q4_k_test.go:15-125 `cQ4_KSource`,
tensor/oracle_q6_k_test.go:15-131 `cQ6_KSource`,
tensor/oracle_c_test.go:16-91 `cQ5_0Source`) and compiles them with gcc at
test time.  This recipe does the same: it reads the Go files as text where
they lie under the reference checkout, writes each C literal to oracle/_ref/
and compiles it with the reference's own flags (oracle_q4_k_test.go:135).
Everything it writes stays in oracle/_ref/ (git-ignored); nothing is copied
into the repository.  Run only where the reference checkout exists.
"""
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "_ref")
REF = os.environ.get("C2SLM_REFERENCE", "/root/reference")

SOURCES = {
    "q4_k": ("tensor/oracle_q4_k_test.go", "cQ4_KSource", ["-O2", "-std=c99", "-pedantic", "-Wall", "-Werror"]),
    "q6_k": ("tensor/oracle_q6_k_test.go", "cQ6_KSource", ["-O2", "-std=c99", "-pedantic", "-Wall", "-Werror"]),
    "q5_0": ("tensor/oracle_c_test.go", "cQ5_0Source", ["-O2"]),
}


def extract(go_path, const_name):
    with open(go_path, "r", encoding="utf-8") as f:
        text = f.read()
    m = re.search(r"const\s+" + re.escape(const_name) + r"\s*=\s*`([^`]*)`", text)
    if not m:
        raise RuntimeError(f"{const_name} not found in {go_path}")
    return m.group(1)


def main():
    if not os.path.isdir(REF):
        print(f"reference checkout {REF} absent: oracle/_ref not built")
        return 0
    os.makedirs(OUT, exist_ok=True)
    for name, (rel, const, flags) in SOURCES.items():
        src = extract(os.path.join(REF, rel), const)
        c_path = os.path.join(OUT, name + ".c")
        with open(c_path, "w", encoding="utf-8") as f:
            f.write(src)
        exe = os.path.join(OUT, name)
        subprocess.run(["gcc", *flags, "-o", exe, c_path, "-lm"], check=True)
        print("built", exe)
    return 0


if __name__ == "__main__":
    sys.exit(main())
