/*
 * CPU oracle for the GGUF block quantizers -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's eager CPU path (the kernels/ modules run
 * under torch on CPU), used by the tests as the parity checker and by the
 * benchmark as the timed CPU baseline. The product path never links, loads or
 * calls it.
 *
 * Every function cites the reference file:line it follows. All arithmetic is
 * IEEE f32 with one rounding per torch op (built with -ffp-contract=off); the
 * reduction orders reproduce what torch 2.10's CPU kernels do for the sums
 * the reference writes (`.sum(-1)`, tree_sum, seq_sum).
 */
#ifndef QS_ORACLE_H
#define QS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (GGUF spec) */
enum {
    QSO_Q4_0 = 2, QSO_Q2_K = 10, QSO_Q3_K = 11, QSO_Q4_K = 12, QSO_Q5_K = 13,
    QSO_Q6_K = 14, QSO_IQ2_XXS = 16, QSO_IQ2_XS = 17, QSO_IQ3_XXS = 18,
    QSO_IQ3_S = 21, QSO_IQ2_S = 22, QSO_IQ4_XS = 23,
    /* no reference module; parity unpinned against the reference */
    QSO_Q4_1 = 3, QSO_Q5_0 = 6, QSO_Q5_1 = 7, QSO_Q8_0 = 8, QSO_IQ4_NL = 20
};

/* bytes of one quantized row of k elements, or -1 for an unsupported type / k */
int64_t qso_row_bytes(int ggml_type, int64_t k);

/* Quantize x (n_rows x k, row-major f32) into out (n_rows * row_bytes bytes).
 * qw: k per-column imatrix weights or NULL. Returns 0, or -1 on bad arguments. */
int qso_quantize(int ggml_type, const float *x, int64_t n_rows, int64_t k,
                 const float *qw, uint8_t *out, int n_threads);

/* Sum helpers exposed for the tests that pin them against torch. */
float qso_sum_cascade8(const float *v, int n);
float qso_sum_tree(const float *v, int n);
uint16_t qso_f32_to_f16(float f);
/* Test hook: plant a known mistake (1..6, see qs_oracle.c); 0 restores the oracle. */
void qso_set_mutation(int m);
/* Square root used for weights: by default the reference's torch.sqrt,
 * reproduced as IEEE sqrtf minus one ulp on a tabulated set (qso_sqrt_ref).
 * Test hooks: another routine (NULL = the default), or plain IEEE sqrtf. */
float qso_sqrt_ref(float v);
void qso_set_sqrt_hook(float (*fn)(float));
void qso_set_sqrt_ieee(int on);
/* Test hook: a per-key rounding table (2^24 int8 ulp offsets from the IEEE
 * root, keyed as qso_sqrt_ref; NULL = off), e.g. torch.sqrt measured on
 * another host. The caller keeps the table alive while it is installed. */
void qso_set_sqrt_table(const int8_t *ulps, int subnormal_ieee);
/* The square root the weights currently use (whichever of the above is set). */
float qso_sqrt(float v);
/* Neighbour list of an off-grid code (tables 0..4: IQ2 256/512/1024, IQ3 256/512):
 * writes up to cap grid indices, returns the list length (0 for on-grid codes). */
int qso_neighbours(int which, int code, uint16_t *out, int cap);
float qso_f16_to_f32(uint16_t h);

#ifdef __cplusplus
}
#endif
#endif
