// Host driver for tests/test_modarith_bounds.py: evaluates the modular
// helpers of fhe-mamba_amd/csrc/modarith.hpp (compiled for the host, the
// same source the kernels use) and the butterflies the NTT kernels build
// from them, on records of little-endian uint64 read from stdin; writes
// one or two uint64 per record to stdout.
//
//   modarith_driver OP < records > results
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "modarith.hpp"

using namespace fhe;

static float rq_of(uint64_t q) {
  // 2^32 / q (1 - 2^-20), rounded down (ModConst::rq of the context).
  const double v = 4294967296.0 / (double)q * (1.0 - 1.0 / 1048576.0);
  float f = (float)v;
  while ((double)f > v) f = nextafterf(f, 0.0f);
  return f;
}

int main(int argc, char** argv) {
  if (argc != 2) return 2;
  const char* op = argv[1];
  struct Op {
    const char* name;
    int in, out;
  } ops[] = {{"shoup_lazy", 2, 1},   {"shoup_lazy4", 2, 1}, {"shoup_lazy4n", 2, 1},
             {"lazy_sub", 2, 1},     {"redc", 2, 1},        {"redc_lazy", 2, 1},
             {"reduce_est", 1, 1},   {"fwd", 3, 2},         {"inv", 3, 2},
             {"fwd_alt_even", 3, 2}, {"fwd_alt_odd", 3, 2}};
  int nin = 0, nout = 0;
  for (const Op& o : ops)
    if (!strcmp(o.name, op)) nin = o.in, nout = o.out;
  if (!nin) return 2;
  // Every record starts with q; the rest are the operands.
  std::vector<uint64_t> rec(nin + 1);
  uint64_t res[2];
  while (fread(rec.data(), 8, nin + 1, stdin) == (size_t)(nin + 1)) {
    const uint64_t q = rec[0], qneg = 0 - q, q4 = 4 * q, q4neg = 0 - 4 * q, q8neg = 0 - 8 * q;
    const uint64_t* a = rec.data() + 1;
    if (!strcmp(op, "shoup_lazy")) {
      res[0] = shoup_lazy(a[0], a[1], host_shoup(a[1], q), q);
    } else if (!strcmp(op, "shoup_lazy4")) {
      res[0] = shoup_lazy4(a[0], a[1], host_shoup(a[1], q), q);
    } else if (!strcmp(op, "shoup_lazy4n")) {
      res[0] = shoup_lazy4n(a[0], a[1], host_shoup(a[1], q), qneg);
    } else if (!strcmp(op, "lazy_sub")) {
      res[0] = lazy_sub(a[0], 0 - a[1]);  // x >= m ? x - m : x with m = a[1]
    } else if (!strcmp(op, "redc")) {
      res[0] = redc(a[0], a[1], q, host_qinv_neg(q));
    } else if (!strcmp(op, "redc_lazy")) {
      res[0] = redc_lazy(a[0], a[1], q, 0 - host_qinv_neg(q));
    } else if (!strcmp(op, "reduce_est")) {
      res[0] = reduce_est(a[0], qneg, rq_of(q));
    } else {
      // Butterflies of the NTT kernels on (x, y, w): forward Cooley-Tukey
      // with X brought below 4q (plain) or 8q (the even stages of the
      // alternating range) or taken as is (its odd stages); inverse
      // Gentleman-Sande with the sum brought below 4q.
      const uint64_t x = a[0], y = a[1], w = a[2], wp = host_shoup(w, q);
      if (!strcmp(op, "inv")) {
        res[1] = shoup_lazy4n(x + q4 - y, w, wp, qneg);
        res[0] = lazy_sub(x + y, q4neg);
      } else {
        const uint64_t X = !strcmp(op, "fwd")            ? lazy_sub(x, q4neg)
                           : !strcmp(op, "fwd_alt_even") ? lazy_sub(x, q8neg)
                                                         : x;
        const uint64_t T = shoup_lazy4n(y, w, wp, qneg);
        res[0] = X + T;
        res[1] = X + q4 - T;
      }
    }
    fwrite(res, 8, nout, stdout);
  }
  return 0;
}
