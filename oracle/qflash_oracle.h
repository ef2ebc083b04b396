/* CPU oracle for the integer attention forward - test infrastructure only. */
#ifndef QFLASH_ORACLE_H
#define QFLASH_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Constants and arithmetic flags of one call (kernel.py:30-36, :302-307). */
typedef struct qfo_params {
    int32_t sm_rscale, exp_M, req_M, l_M, acc_M;
    int32_t exp_use_shift, l_use_shift, acc_use_shift, l_shift, acc_shift;
} qfo_params;

/* strides: 20 element strides, (z,h,n,d) for q, k, v, o, bias (bias may be
 * NULL; its strides may be 0 for broadcast).  Heads zh in [zh_begin, zh_end)
 * are computed (zh_end <= 0 means all).  Returns 0 or a negative code. */
int qfo_attention_codes(const int8_t* q, const int8_t* k, const int8_t* v, int8_t* o, const int32_t* bias,
                        const int64_t* strides, int Z, int H, int N, int D, const qfo_params* p,
                        int n_threads, int zh_begin, int zh_end);

void qfo_exp2_requant(const int32_t* x, int32_t* e, int32_t* pq, int64_t n, const qfo_params* p);
void qfo_release_n(const int32_t* x, const int32_t* alpha, int32_t* out, int64_t n, int32_t M, int32_t shift,
                   int use_shift, int32_t rs);

#ifdef __cplusplus
}
#endif
#endif
