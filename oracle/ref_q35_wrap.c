/*
 * ref_q35_wrap.c -- exposes the file-static INT4/INT8 GEMVs of the reference's src/eif_qwen35.c
 * (int4_gemv :293-352, int8_gemv :384-419) by compiling that file where it lies, the way the reference's own
 * tests/test_q35_int4.c:3 reaches them. Built only into oracle/_ref/libref.so (test infrastructure); the path
 * of the reference tree comes from the Makefile's -DREF_QWEN35_C.
 */
#include REF_QWEN35_C

void ref_q35_int4_gemv(float *out, const uint8_t *W, const float *sc, const float *x, int rows, int cols)
{
    int4_gemv(out, W, sc, x, rows, cols);
}

void ref_q35_int8_gemv(float *out, const int8_t *W, const float *sc, const float *x, int rows, int cols)
{
    int8_gemv(out, W, sc, x, rows, cols);
}
