/*
 * Which float64 library results can round to a different float32 between
 * two libraries?  The reference computes
 *   softmax    e = float32(math.Exp(float64(x - max)))       (tensor/ops.go:330)
 *   RoPE table cos/sin = float32(math.Cos/Sin(p * 1/math.Pow(theta, 2i/hd)))
 *                                                            (tensor/ops.go:237-257)
 * with Go's math package; the oracle and this build use glibc (host) and the
 * HIP device library.  For every input this program computes the exact
 * value in long double (64-bit mantissa) and its distance to the nearest
 * float32 rounding boundary (the midpoint of two neighbouring floats).  An
 * input is stable when that distance exceeds the error band of two float64
 * libraries of the stated accuracy: then both round to the same float32.
 *
 *   exp:  every float32 t <= 0 with exp(t) >= 2^-150 (smaller results are
 *         0 in float32 for any library); band = 2 ulp_f64 of the result
 *         (a library within 1 ulp, plus margin).
 *   RoPE: p in [0, P), i in [0, hd/2).  pow within k ulp gives freq and
 *         val = p*freq within (k+1) ulp relative, so cos/sin move by
 *         |sin or cos| * val * (k+1) * 2^-52; band = that + 2 ulp_f64.
 *         Reported for k = 1 and k = 4.  i = 0 has freq = 1 exactly.
 *
 * Output (stdout): one line per exception and summary lines; see
 * tests/test_f32_stability.py.
 *
 * Build: gcc -O2 -fopenmp -o f32_stability f32_stability.c -lm
 * Usage: f32_stability exp | f32_stability rope P HD THETA
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* distance from v (> 0) to the nearest float32 rounding midpoint */
static long double mid_dist(long double v) {
  float f = (float)v;                       /* round to nearest */
  long double lf = f;
  float up = nextafterf(f, INFINITY), dn = nextafterf(f, 0.0f);
  long double m1 = ((long double)f + (long double)up) / 2, m0 = ((long double)f + (long double)dn) / 2;
  long double d1 = fabsl(v - m1), d0 = fabsl(v - m0);
  (void)lf;
  return d1 < d0 ? d1 : d0;
}

static long double ulp64(long double v) {
  v = fabsl(v);
  if (v == 0) return 0x1p-1074L;
  int e = ilogbl(v);
  if (e < -1022) e = -1022;
  return ldexpl(1.0L, e - 52);
}

static int run_exp(void) {
  /* t from -0 down to the first float with exp(t) < 2^-150 */
  const long double lo = 0x1p-150L;
  long n_exc = 0, n_all = 0;
  /* negative floats order by magnitude with their bit patterns, so the last
     t with exp(t) >= 2^-150 is found by bisection */
  uint32_t last = 0x80000000u, bad = 0xc3000000u; /* exp(-0) = 1; exp(-128) < 2^-150 */
  while (bad - last > 1) {
    uint32_t mid = last + (bad - last) / 2;
    if (expl((long double)bits_f(mid)) >= lo) last = mid; else bad = mid;
  }
#pragma omp parallel for schedule(dynamic, 1 << 20) reduction(+ : n_exc, n_all)
  for (int64_t u = 0x80000000ll; u <= (int64_t)last; ++u) {
    float t = bits_f((uint32_t)u);
    long double v = expl((long double)t);
    n_all++;
    if (v == 1.0L) continue; /* exp(-0) = 1 exactly */
    if (mid_dist(v) <= 2 * ulp64(v)) {
      n_exc++;
      double g = exp((double)t); /* this host's float64 library, for the record */
#pragma omp critical
      printf("exp t=0x%08x (%.9g) exact_f32=0x%08x glibc_f32=0x%08x\n", (uint32_t)u, (double)t,
             f_bits((float)v), f_bits((float)g));
    }
  }
  printf("exp inputs %ld exceptions %ld last_t=0x%08x\n", n_all, n_exc, last);
  return 0;
}

static int run_rope(int P, int hd, double theta) {
  long exc1 = 0, exc4 = 0, n_all = 0;
  int min_p1 = P, min_p4 = P;
  int half = hd / 2;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : exc1, exc4, n_all) reduction(min : min_p1, min_p4)
  for (int p = 0; p < P; ++p) {
    for (int i = 0; i < half; ++i) {
      long double F = (i == 0) ? 1.0L : 1.0L / powl((long double)theta, (long double)(2 * i) / (long double)hd);
      long double val = (long double)p * F;
      long double c = cosl(val), s = sinl(val);
      for (int which = 0; which < 2; ++which) {
        long double v = which ? s : c, other = which ? c : s;
        n_all++;
        if (v == 0) continue; /* p = 0: sin = 0 and cos = 1 exactly */
        long double av = fabsl(v);
        long double d = mid_dist(av);
        long double prop1 = (i == 0) ? 0 : fabsl(other) * val * 2 * 0x1p-52L;
        long double prop4 = (i == 0) ? 0 : fabsl(other) * val * 5 * 0x1p-52L;
        int e1 = d <= prop1 + 2 * ulp64(av), e4 = d <= prop4 + 2 * ulp64(av);
        exc1 += e1;
        exc4 += e4;
        if (e1 && p < min_p1) min_p1 = p;
        if (e4 && p < min_p4) min_p4 = p;
        if (e1) {
#pragma omp critical
          printf("rope k1 p=%d i=%d %s exact_f32=0x%08x\n", p, i, which ? "sin" : "cos", f_bits((float)v));
        }
      }
    }
  }
  printf("rope entries %ld exceptions_k1 %ld exceptions_k4 %ld first_p_k1 %d first_p_k4 %d\n", n_all, exc1, exc4,
         min_p1, min_p4);
  return 0;
}

int main(int argc, char** argv) {
  if (argc >= 2 && !strcmp(argv[1], "exp")) return run_exp();
  if (argc >= 5 && !strcmp(argv[1], "rope")) return run_rope(atoi(argv[2]), atoi(argv[3]), atof(argv[4]));
  fprintf(stderr, "usage: %s exp | rope P HD THETA\n", argv[0]);
  return 2;
}
