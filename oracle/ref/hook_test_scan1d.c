/* Exposes the C restatement of the forward scan that lives inside the
 * reference's unit test tests/unit/test_scan1d.c:33-68 (scan1d_ref: the asm
 * recurrence without clamp, full h history [L, D, M], zero initial state) so
 * the oracle can be compared with it bit for bit.
 *
 * The reference test source is compiled in place: this file includes it from
 * the reference tree at build time and nothing is copied into the
 * repository. Its main() is renamed, kept local by the export map and
 * garbage-collected, so the scan1d symbol it would call is never linked and
 * nothing stands in for the reference's NASM code. */
#define main kmr_unused_main_test_scan1d
#include REF_TEST_FILE
#undef main

void kmr_test_scan1d_ref(const float *x, const float *A, const float *B,
                         const float *C, const float *delta, float *h, float *y,
                         long L, long D, long M) {
    scan1d_ref(x, A, B, C, delta, h, y, L, D, M);
}
