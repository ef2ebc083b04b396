/*
 * CPU oracle for the integer-only attention forward, in plain C (OpenMP).
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/ as the checker at full sizes, by
 * __graft_entry__.smoke() as the checker, and by bench.py's cpu_baseline leg
 * (kind "port").  The product library never links or calls it.
 *
 * Restates qflash_kernel / qflash_masked_kernel of EfficientCompLab/qflash
 * (qflash/kernel.py:85-180, :183-272) with Triton's arithmetic rules:
 *   - int32 tensors wrap (two's complement);
 *   - `>>` on int32 clamps: a shift count read as unsigned >= 32 gives the
 *     sign fill (numpy right_shift, what the Triton interpreter runs);
 *   - integer `//` truncates toward zero;
 *   - int/int `/` is fp32 true division; fp32 -> int32 truncates and yields
 *     INT32_MIN for NaN / inf / out of range (x86 cvttss2si, numpy astype);
 *   - `.to(tl.int8)` keeps the low byte.
 * One row's result depends only on that row, processed 32 key columns per
 * step in order (BLOCK_N = 32, kernel.py:26-27).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "qflash_oracle.h"

#define QFO_NEG_INF (-(1 << 20)) /* kernel.py:137 */
#define QFO_BN 32                /* kernel.py:27 */

static inline int32_t w32(int64_t x) { return (int32_t)(uint32_t)(uint64_t)x; }

/* clamping arithmetic shift right of an int32 by an int32 count */
static inline int32_t sra32(int32_t a, int32_t b) {
    uint32_t ub = (uint32_t)b;
    if (ub >= 32u) return a < 0 ? -1 : 0;
    return a >> ub;
}

static inline int32_t tdiv32(int32_t a, int32_t b) {
    /* C division truncates; INT32_MIN / -1 (sm_rscale = -1) wraps to INT32_MIN as numpy's int32 does */
    return (int32_t)((int64_t)a / (int64_t)b);
}

/* exp2_i32, kernel.py:40-59 */
static inline int32_t qfo_exp2(int32_t x, const qfo_params* p) {
    int32_t rs = p->sm_rscale, q;
    if (p->exp_use_shift)
        q = sra32(w32((int64_t)x * p->exp_M), 16);
    else
        q = tdiv32(w32(-(int64_t)x), rs);
    int32_t r = w32((int64_t)x + w32((int64_t)q * rs));
    return sra32(w32((int64_t)sra32(r, 1) + rs), q);
}

/* requantize, kernel.py:62-64 */
static inline int32_t qfo_requant(int32_t e, const qfo_params* p) {
    int32_t t = sra32(w32((int64_t)w32((int64_t)e * p->req_M) + (1 << 15)), 16);
    return (int32_t)(int8_t)(uint8_t)(uint32_t)t;
}

/* scale_release, kernel.py:67-82 */
static inline int32_t qfo_release(int32_t x, int32_t alpha, int32_t M, int32_t shift, int use_shift,
                                  int32_t rs) {
    if (use_shift) {
        uint64_t prod = (uint64_t)((int64_t)x * (int64_t)alpha) * (uint64_t)(int64_t)M;
        prod += (uint64_t)1 << (shift - 1);
        return w32(((int64_t)prod) >> shift);
    }
    return tdiv32(w32((int64_t)x * alpha), rs);
}

static inline int32_t cvt_x86(float f) {
    if (!(f >= -2147483648.0f && f < 2147483648.0f)) return INT32_MIN;
    return (int32_t)f;
}

/* int8 dot product of length D with element strides (hot loop of the port) */
static inline int32_t dot_i8(const int8_t* a, int64_t sa, const int8_t* b, int64_t sb, int D) {
    int32_t s = 0;
    if (sa == 1 && sb == 1) {
        for (int d = 0; d < D; ++d) s += (int32_t)a[d] * (int32_t)b[d];
    } else {
        for (int d = 0; d < D; ++d) s += (int32_t)a[d * sa] * (int32_t)b[d * sb];
    }
    return s;
}

__attribute__((target_clones("avx2", "default")))
static void qfo_row(const int8_t* qrow, int64_t sqd, const int8_t* kb, int64_t skn, int64_t skd,
                    const int8_t* vt /* D x Npad, contiguous transpose of V */, int Npad,
                    const int32_t* brow, int64_t sbn, int8_t* orow, int64_t sod, int N, int D,
                    const qfo_params* p, int32_t* acc) {
    const int masked = brow != NULL;
    const int pad_cols = masked || (N % QFO_BN) != 0; /* kernel.py:106 */
    int32_t m = QFO_NEG_INF, l = 1;                    /* kernel.py:138-139 */
    for (int d = 0; d < D; ++d) acc[d] = 0;            /* kernel.py:140 */
    int32_t s[QFO_BN], pj[QFO_BN];
    for (int start = 0; start < N; start += QFO_BN) {  /* kernel.py:147 */
        int32_t mx = INT32_MIN;
        for (int jj = 0; jj < QFO_BN; ++jj) {
            int j = start + jj;
            int32_t val;
            if (j < N) {
                val = dot_i8(qrow, sqd, kb + (int64_t)j * skn, skd, D); /* :153 */
                if (masked) val = w32((int64_t)val + brow[(int64_t)j * sbn]); /* :253 */
            } else {
                val = pad_cols ? QFO_NEG_INF : 0; /* :155-156 */
            }
            s[jj] = val;
            if (val > mx) mx = val;
        }
        int32_t mn = m > mx ? m : mx; /* :158 */
        int32_t lij = 0;
        for (int jj = 0; jj < QFO_BN; ++jj) { /* :159-162 */
            pj[jj] = qfo_requant(qfo_exp2(w32((int64_t)s[jj] - mn), p), p);
            lij += pj[jj];
        }
        int32_t alpha = qfo_exp2(w32((int64_t)m - mn), p); /* :163 */
        l = w32((int64_t)qfo_release(l, alpha, p->l_M, p->l_shift, p->l_use_shift, p->sm_rscale) + lij);
        int nv = N - start < QFO_BN ? N - start : QFO_BN;
        for (int d = 0; d < D; ++d) { /* :165, :171 */
            int32_t a = qfo_release(acc[d], alpha, p->acc_M, p->acc_shift, p->acc_use_shift, p->sm_rscale);
            const int8_t* vr = vt + (int64_t)d * Npad + start;
            int32_t t = 0;
            for (int jj = 0; jj < nv; ++jj) t += pj[jj] * (int32_t)vr[jj];
            acc[d] = w32((int64_t)a + t);
        }
        m = mn; /* :172 */
    }
    float lf = (float)l;
    for (int d = 0; d < D; ++d) { /* :176-178 */
        float qf = (float)acc[d] / lf;
        orow[(int64_t)d * sod] = (int8_t)(uint8_t)(uint32_t)cvt_x86(qf);
    }
}

int qfo_attention_codes(const int8_t* q, const int8_t* k, const int8_t* v, int8_t* o, const int32_t* bias,
                        const int64_t* st, int Z, int H, int N, int D, const qfo_params* p,
                        int n_threads, int zh_begin, int zh_end) {
    if (!q || !k || !v || !o || !st || !p || Z <= 0 || H <= 0 || N <= 0 || D <= 0) return -1;
    if (p->sm_rscale == 0) return -2; /* the reference's host raises before any launch with rs = 0 */
    if (p->l_use_shift && (p->l_shift < 1 || p->l_shift > 62)) return -3;
    if (p->acc_use_shift && (p->acc_shift < 1 || p->acc_shift > 62)) return -3;
    if (zh_end <= 0 || zh_end > Z * H) zh_end = Z * H;
    if (zh_begin < 0) zh_begin = 0;
    const int Npad = (N + QFO_BN - 1) / QFO_BN * QFO_BN;
    int rc = 0;
#pragma omp parallel num_threads(n_threads > 0 ? n_threads : 1)
    {
        int8_t* vt = (int8_t*)calloc((size_t)D * Npad, 1);
        int32_t* acc = (int32_t*)malloc(sizeof(int32_t) * (size_t)D);
        if (!vt || !acc) {
#pragma omp atomic write
            rc = -4;
        }
#pragma omp for schedule(dynamic, 1)
        for (int zh = zh_begin; zh < zh_end; ++zh) {
            if (!vt || !acc) continue;
            int z = zh / H, h = zh % H;
            const int8_t* qb = q + z * st[0] + h * st[1];
            const int8_t* kb = k + z * st[4] + h * st[5];
            const int8_t* vb = v + z * st[8] + h * st[9];
            int8_t* ob = o + z * st[12] + h * st[13];
            for (int j = 0; j < N; ++j)
                for (int d = 0; d < D; ++d) vt[(int64_t)d * Npad + j] = vb[j * st[10] + d * st[11]];
            for (int i = 0; i < N; ++i) {
                const int32_t* brow = bias ? bias + z * st[16] + h * st[17] + i * st[18] : NULL;
                qfo_row(qb + i * st[2], st[3], kb, st[6], st[7], vt, Npad, brow, st[19],
                        ob + i * st[14], st[15], N, D, p, acc);
            }
        }
        free(vt);
        free(acc);
    }
    return rc;
}

/* Primitive entry points so tests can sweep them exhaustively against numpy. */
void qfo_exp2_requant(const int32_t* x, int32_t* e, int32_t* pq, int64_t n, const qfo_params* p) {
    for (int64_t i = 0; i < n; ++i) {
        e[i] = qfo_exp2(x[i], p);
        pq[i] = qfo_requant(e[i], p);
    }
}

void qfo_release_n(const int32_t* x, const int32_t* alpha, int32_t* out, int64_t n, int32_t M, int32_t shift,
                   int use_shift, int32_t rs) {
    for (int64_t i = 0; i < n; ++i) out[i] = qfo_release(x[i], alpha[i], M, shift, use_shift, rs);
}
