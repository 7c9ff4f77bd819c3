/*
 * moe_oracle.c -- CPU restatement of the Mixtral MoE python_vm arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP kernel is
 * compared against (and the CPU baseline the benchmark times); nothing in the
 * product path may link or call it.
 *
 * It restates, rounding point by rounding point, the torch CPU computation of
 *   megakernels/demos/latency/python_vm.py:29-56   (matvec, rms_norm)
 *   megakernels/mixtral/python_vm.py:228-277        (opcode 5)
 *   megakernels/mixtral/python_vm.py:284-314        (opcode 6)
 *   megakernels/mixtral/python_vm.py:356-371        (opcode 8, router part)
 * on bf16 values stored as uint16 bit patterns:
 *   - bf16 -> fp32 is exact (bits << 16); fp32 -> bf16 rounds to nearest
 *     even with NaN -> 0x7fc0, the conversion torch applies on every
 *     `.to(bfloat16)` and on every bf16 elementwise result;
 *   - a bf16 matvec row (torch einsum "o i, i -> o" on bf16) is an fp32
 *     accumulation of exact bf16 x bf16 products, rounded once to bf16.  Here
 *     16 fp32 partial sums in fixed lane order are combined in double, so the
 *     result is independent of thread count;
 *   - fp32 reductions the reference does in fp32 (mean of squares, router
 *     logits) are accumulated in double and rounded once to fp32.
 * Softmax, top-k and the score renormalisation are done by the Python glue
 * with torch's own fp32 routines, as the reference does.
 *
 * Build: oracle/Makefile (gcc, OpenMP).  Row loops are parallel over rows;
 * each row is computed by one thread in a fixed order.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bf2f(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline uint16_t f2bf(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

static inline float rbf(float f) { return bf2f(f2bf(f)); }

/* fp32-accumulated dot product of two bf16 vectors of length n. */
static double dot_bf16(const uint16_t *a, const uint16_t *b, int64_t n) {
    float part[16];
    for (int l = 0; l < 16; ++l) part[l] = 0.0f;
    int64_t i = 0;
    for (; i + 16 <= n; i += 16)
        for (int l = 0; l < 16; ++l) part[l] += bf2f(a[i + l]) * bf2f(b[i + l]);
    double s = 0.0;
    for (int l = 0; l < 16; ++l) s += (double)part[l];
    for (; i < n; ++i) s += (double)(bf2f(a[i]) * bf2f(b[i]));
    return s;
}

void orc_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int orc_get_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* lat/python_vm.py:50-56: out = bf16(w * bf16(x * rsqrt(mean(x^2) + eps))). */
void orc_rms_norm(const uint16_t *x, const uint16_t *w, int64_t n, float eps, uint16_t *out) {
    double ss = 0.0;
    for (int64_t i = 0; i < n; ++i) {
        const float v = bf2f(x[i]);
        ss += (double)(v * v);
    }
    const float var = (float)(ss / (double)n);
    const float r = 1.0f / sqrtf(var + eps);
    for (int64_t i = 0; i < n; ++i) {
        const float nv = rbf(bf2f(x[i]) * r);
        out[i] = f2bf(bf2f(w[i]) * nv);
    }
}

/* mkm/python_vm.py:245: logits[e] = W_r[e].float() @ normed.float() (+ bias). */
void orc_router_logits(const uint16_t *wr, const uint16_t *normed, int64_t E, int64_t H, const float *bias,
                       float *logits) {
    for (int64_t e = 0; e < E; ++e) {
        double s = 0.0;
        const uint16_t *row = wr + e * H;
        for (int64_t i = 0; i < H; ++i) s += (double)bf2f(row[i]) * (double)bf2f(normed[i]);
        float l = (float)s;
        if (bias) l += bias[e];
        logits[e] = l;
    }
}

/* mkm/python_vm.py:258-275 for rows [row0, row0 + nrows) of one expert:
 *   g = bf16(Wg[r] . normed), u = bf16(Wu[r] . normed)
 *   out[r - row0] = bf16(bf16(silu(g)) * u),  silu(g) = g / (1 + exp(-g)). */
void orc_upgate_silu(const uint16_t *gate, const uint16_t *up, const uint16_t *normed, int64_t H, int64_t row0,
                     int64_t nrows, uint16_t *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < nrows; ++i) {
        const int64_t r = row0 + i;
        const float g = rbf((float)dot_bf16(gate + r * H, normed, H));
        const float u = rbf((float)dot_bf16(up + r * H, normed, H));
        const float sg = rbf(g / (1.0f + expf(-g)));
        out[i] = f2bf(sg * u);
    }
}

/* mkm/python_vm.py:296-310 for one expert slot over rows [row0, row0+nrows):
 *   o = bf16(Wd[r] . act);  hidden[r] = bf16(hidden[r] + bf16(score * o)). */
void orc_down_accumulate(const uint16_t *down, const uint16_t *act, int64_t F, int64_t row0, int64_t nrows,
                         float score, uint16_t *hidden) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < nrows; ++i) {
        const int64_t r = row0 + i;
        const float o = rbf((float)dot_bf16(down + r * F, act, F));
        const float add = rbf(score * o);
        hidden[r] = f2bf(bf2f(hidden[r]) + add);
    }
}

/* Plain bf16 matvec rows (lat/python_vm.py:29-47): out[i] = bf16(M[row0+i] . v)
 * over K columns; rows are `ld` elements apart (ld > K for a column block of
 * a wider matrix, as the LM head's 2048-column reduction blocks are). */
void orc_matvec(const uint16_t *mat, int64_t ld, const uint16_t *vec, int64_t K, int64_t row0, int64_t nrows,
                uint16_t *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < nrows; ++i) out[i] = f2bf((float)dot_bf16(mat + (row0 + i) * ld, vec, K));
}

/* Exported conversions so tests can pin the rounding helpers themselves. */
uint16_t orc_f32_to_bf16(float f) { return f2bf(f); }
float orc_bf16_to_f32(uint16_t h) { return bf2f(h); }
