"""The quantiser's d = amax/127 (the product with RN(1/127) corrected by its
exact fma residual, div127 in c2slm_amd/csrc/c2h_kernels.hip) equals the
IEEE quotient of internal/simd/c2_quantize_q8_k_gen.go:40-47.  The same
formula in C (glibc's fmaf is correctly rounded, like v_fma_f32) is swept
over the non-negative floats: every subnormal and the binades around the
quantiser's usual amax fully, the rest with a stride; +Inf maps to +Inf.
(A full sweep of all 2^31 values found no mismatch; it takes about 40 s.)"""
import subprocess
import textwrap

SRC = textwrap.dedent(r"""
    #include <math.h>
    #include <stdint.h>
    #include <stdio.h>
    #include <string.h>
    static float div127(float m) {
      const float C = 1.0f / 127.0f;
      float q0 = m * C;
      float r = fmaf(-q0, 127.0f, m);
      float q1 = fmaf(r, C, q0);
      return (m == INFINITY) ? m : q1;
    }
    static int check(uint32_t lo, uint32_t hi, uint32_t step, unsigned long long* n) {
      for (uint64_t u = lo; u <= hi; u += step) {
        float m;
        uint32_t b = (uint32_t)u;
        memcpy(&m, &b, 4);
        volatile float want = m / 127.0f;
        float got = div127(m);
        ++*n;
        if (memcmp(&got, (const void*)&want, 4)) { printf("mismatch 0x%08x\n", b); return 1; }
      }
      return 0;
    }
    int main(void) {
      unsigned long long n = 0;
      int bad = check(0u, 0x00800000u, 1, &n);                 /* zero and subnormals */
      bad |= check(0x3c000000u, 0x43800000u, 1, &n);          /* 2^-7 .. 256 */
      bad |= check(0x00800000u, 0x7f7fffffu, 61, &n);         /* all binades, strided */
      bad |= check(0x7f7fffffu, 0x7f800000u, 1, &n);          /* FLT_MAX, +Inf */
      printf("%llu values\n", n);
      return bad;
    }
""")


def test_div127_matches_ieee_quotient(tmp_path):
    c = tmp_path / "div127.c"
    c.write_text(SRC)
    exe = tmp_path / "div127"
    subprocess.run(["gcc", "-O2", "-o", str(exe), str(c), "-lm"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout
