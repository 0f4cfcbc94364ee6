// host_check.hip -- host-only check of the library's planning code under
// AddressSanitizer / UndefinedBehaviorSanitizer (built by `make host-check`
// with --offload-host-only: no device code, no GPU needed, nothing launched).
//
// Every backward composition is run in its sizing mode (the same dispatch as
// a real call: algorithm choice, stride phases, weight-gradient plans,
// split-K plans, im2col sizes; it stops before any launch) over a grid of
// shapes, dtypes and algorithms, together with the algorithm selectors and the
// shape checks of the entry points.  A sanitizer report or a bad size fails.
#include "vh_api.hip"

#include <cstdio>

int main() {
  using namespace vh;
  long n = 0, fails = 0;
  const long Bs[] = {1, 2, 3, 16, 128};
  const long Cs[] = {1, 3, 16, 27, 64, 256};
  const long Hs[] = {1, 5, 14, 28, 56, 256};
  const long Ks[] = {1, 3, 5, 7};
  const long Ss[] = {1, 2, 3, 4, 5};
  char dummy[64];
  const void* p = dummy;
  for (long B : Bs)
    for (long C : Cs)
      for (long O : Cs)
        for (long H : Hs)
          for (long K : Ks)
            for (long S : Ss)
              for (long P = 0; P <= K; P += (K > 2 ? K / 2 : 1)) {
                if (B * C * H * H > (1L << 26) || B * O * H * H > (1L << 26)) continue;
                for (int dt : {(int)VH_F32, (int)VH_BF16})
                  for (int algo : {(int)VH_ALGO_DIRECT, (int)VH_ALGO_IM2COL, (int)VH_ALGO_IGEMM}) {
                    size_t need = (size_t)-1;
                    const int st = conv2d_backward_impl(dt, algo, p, p, p, (void*)p, (void*)p, (void*)p, B, C, O,
                                                        H, H, K, K, S, S, P, P, nullptr, false, &need);
                    ++n;
                    // valid geometry must plan (sizes below 2^31 elements); invalid must be rejected
                    const bool geom_ok = H + 2 * P >= K;
                    if (geom_ok && st != VH_OK && st != VH_ERR_UNSUPPORTED) {
                      printf("unexpected status %d: B%ld C%ld O%ld H%ld K%ld S%ld P%ld dt%d algo%d: %s\n", st, B, C,
                             O, H, K, S, P, dt, algo, g_err);
                      ++fails;
                    }
                    if (!geom_ok && st == VH_OK) {
                      printf("accepted bad geometry B%ld C%ld H%ld K%ld P%ld\n", B, C, H, K, P);
                      ++fails;
                    }
                    if (st == VH_OK && need == (size_t)-1) {
                      printf("no size: B%ld C%ld O%ld H%ld K%ld S%ld P%ld\n", B, C, O, H, K, S, P);
                      ++fails;
                    }
                  }
                (void)vh_conv_algo_auto_select(B, C, H, H, K, 1);
                (void)vh_conv_algo_auto_select(B, C, H, H, K, 0);
                (void)vh_conv_algo_select_mi355x(B, C, O, H, H, K, K, S, S, P, P);
              }
  // shape checks of the entry points' validation (negative, zero, overflow)
  ConvDims bad[] = {{-1, 1, 1, 4, 4, 3, 3, 1, 1, 1, 1, 4, 4},
                    {1, 0, 1, 4, 4, 3, 3, 1, 1, 1, 1, 4, 4},
                    {1, 1, 1, 4, 4, 3, 3, 0, 1, 1, 1, 4, 4},
                    {1, 1, 1, 4, 4, 3, 3, 1, 1, -1, 1, 4, 4},
                    {1, 1, 1, 4, 4, 3, 3, 1, 1, 1, 1, 5, 4},
                    {1L << 20, 1L << 10, 1, 64, 64, 3, 3, 1, 1, 1, 1, 64, 64}};
  for (const ConvDims& d : bad) {
    ++n;
    if (check_conv(d, true) == VH_OK) {
      printf("check_conv accepted a bad shape (B%ld C%ld SH%ld PH%ld HO%ld)\n", d.B, d.C, d.SH, d.PH, d.HO);
      ++fails;
    }
  }
  printf("host_check: %ld plans, %ld failures\n", n, fails);
  return fails ? 1 : 0;
}
