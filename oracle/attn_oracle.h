/* attn_oracle.h — CPU oracle of the FlashAttention-2 forward.
 * TEST INFRASTRUCTURE ONLY (see attn_oracle.c); not part of the product. */
#ifndef ATTN_ORACLE_H
#define ATTN_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORACLE_F16 = 0, ORACLE_BF16 = 1 };

/* Planted mistakes, used only by the tests that show the pinning checks catch
 * them.  0 = the oracle proper. */
enum {
  ORACLE_MUT_NONE = 0,
  ORACLE_MUT_NO_SCALE = 1,       /* softmax scale dropped                   */
  ORACLE_MUT_CAUSAL_DIAG = 2,    /* causal mask also hides the diagonal     */
  ORACLE_MUT_LSE_NO_MAX = 3,     /* LSE forgets the max term                */
  ORACLE_MUT_TRANSPOSE_S = 4,    /* scores transposed: s_ij = q_j . k_i     */
  ORACLE_MUT_NO_NORMALISE = 5    /* O not divided by the row sum            */
};

int oracle_attn_f64(const float* q, const float* k, const float* v, double* o, double* lse, int B,
                    int H, int N, int D, double scale, int causal, int mutation);

int oracle_attn_rows_f64(const float* q, const float* k, const float* v, int B, int H, int N,
                         int D, double scale, int causal, int mutation, const int32_t* sel_bh,
                         const int32_t* sel_row, int64_t n_sel, double* o_sel, double* lse_sel);

int oracle_ref_online_f32(const float* q, const float* k, const float* v, float* o, int B, int H,
                          int N, int D, float scale, int causal, int64_t row_begin,
                          int64_t row_end);

int oracle_kernel_numerics(const float* q, const float* k, const float* v, float* o, float* lse,
                           int B, int H, int N, int D, float scale, int causal, int dtype,
                           int block_n);

int oracle_kernel_numerics_rows(const float* q, const float* k, const float* v, int B, int H,
                                int N, int D, float scale, int causal, int dtype, int block_n,
                                const int32_t* sel_bh, const int32_t* sel_row, int64_t n_sel,
                                float* o_sel, float* lse_sel);
void oracle_round_f16(const float* in, float* out, uint16_t* bits, int64_t n);
void oracle_round_bf16(const float* in, float* out, uint16_t* bits, int64_t n);

int oracle_num_threads(void);
void oracle_set_num_threads(int n);

#ifdef __cplusplus
}
#endif

#endif
