/* Exposes scan_forward_ref from the reference's unit test
 * tests/unit/test_scan1d_backward.c:28-60 (a second in-test restatement of
 * the forward recurrence) for bit-for-bit comparison with the oracle. The
 * test source is compiled in place from the reference tree; its main() is
 * renamed, kept local and garbage-collected. */
#define main kmr_unused_main_test_scan1d_backward
#include REF_TEST_FILE
#undef main

void kmr_test_scan1d_backward_forward_ref(const float *x, const float *A, const float *B,
                                          const float *C, const float *delta, float *h,
                                          float *y, long L, long D, long M) {
    scan_forward_ref(x, A, B, C, delta, h, y, L, D, M);
}
