/*
 * CPU oracle for the layer-streaming path: a plain scalar C restatement of
 * the reference's arithmetic.  TEST INFRASTRUCTURE ONLY -- tests, the smoke
 * check and the benchmark's CPU-baseline leg may call it, to check results;
 * the product never links or loads it.
 *
 * Built by oracle/Makefile with -ffp-contract=off so that every operation
 * below is exactly one IEEE-rounded step as written.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* fp32 -> bf16 cast.  Follows the reference's CPU cast,
 * layer_state.py:301 (`bf16_buf.copy_(fp32_master)`), which runs torch's
 * vectorised conversion: round to nearest even on the bit pattern
 * (add 0x7FFF plus the lowest kept bit, keep the high half) and 0xFFFF for
 * every NaN. */
static uint16_t rne(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0xFFFFu;
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

void oracle_cast_f32_bf16(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = rne(src[i]);
}

/* fp32 -> fp16, for units of dtype float16: the same cast of
 * layer_state.py:301 into a float16 convert buffer (torch's CPU conversion):
 * IEEE round to nearest even with subnormals, overflow to infinity, NaN ->
 * quiet NaN keeping the sign and the top 9 payload bits.  Written from the
 * IEEE definition: scale to units of the result's last place, round. */
static uint16_t rne_f16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x1FFu));
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    const int e = (int)(a >> 23);                 /* biased fp32 exponent */
    if (e == 0) return sign;                      /* fp32 zero or subnormal: far below 2^-24 */
    const uint32_t m = (a & 0x7FFFFFu) | 0x800000u;
    /* value = m * 2^(e-150); the half's unit in the last place is 2^-24 below
     * 2^-14 and 2^(e-127-10) above it */
    const int ulp_exp = e >= 113 ? e - 137 : -24;
    const int shift = ulp_exp - (e - 150);        /* bits of m below that unit */
    if (shift > 31) return sign;
    uint32_t q = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    if (e >= 113) {
        /* q is 1.mantissa in [2^10, 2^11]; a carry to 2^11 moves to the next binade */
        return (uint16_t)(sign | ((((uint32_t)(e - 112)) << 10) + (q - 0x400u)));
    }
    return (uint16_t)(sign | q);                  /* subnormal, or 0x400 = the smallest normal */
}

void oracle_cast_f32_f16(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = rne_f16(src[i]);
}

/* bf16 -> fp32 widening: the `.float()` of layer_adam.py:404. */
void oracle_widen_bf16(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        uint32_t u = (uint32_t)src[i] << 16;
        memcpy(&dst[i], &u, 4);
    }
}

/* Pack: concatenate segments (the flat layout of layer_state.py:241-264,
 * where view k starts at the sum of the sizes of the views before it). */
void oracle_pack_b16(const uint16_t* const* srcs, const size_t* ns, int nsegs, uint16_t* dst) {
    size_t off = 0;
    for (int k = 0; k < nsegs; ++k) {
        memcpy(dst + off, srcs[k], ns[k] * sizeof(uint16_t));
        off += ns[k];
    }
}

/* ------------------------------------------------------------------ */
/* AdamW.  State and scalars follow Adam_Optimizer,
 * optimizer/layer_adam/csrc/cpu_adam.h:26-106:
 *   IncrementStep  cpu_adam.h:57-76   (beta^t: float product when the step
 *                                      advances by one, else pow in double)
 *   update_state   cpu_adam.h:77-89   (bc1 = 1 - beta1^t,
 *                                      bc2 = 1 / sqrt(1 - beta2^t), float)
 * Per element, the vector body Step_AVX cpu_adam.h:170-191 and, for the
 * last n % 16 elements of a call, the scalar tail cpu_adam_impl.cpp:45-64
 * as the reference's compiler contracts it. */
typedef struct oracle_adam {
    float alpha, beta1, beta2, eps, weight_decay;
    float beta1_t, beta2_t;
    size_t step;
    int adamw_mode;
    float bc1, bc2;
} oracle_adam;

void oracle_adam_init(oracle_adam* s, float alpha, float b1, float b2, float eps, float wd,
                      int adamw_mode) {
    s->alpha = alpha;
    s->beta1 = b1;
    s->beta2 = b2;
    s->eps = eps;
    s->weight_decay = wd;
    s->beta1_t = 1.0f;
    s->beta2_t = 1.0f;
    s->step = 0;
    s->adamw_mode = adamw_mode;
    s->bc1 = 1.0f;
    s->bc2 = 1.0f;
}

static void increment_step(oracle_adam* s, size_t step, float b1, float b2) {
    if (b1 != s->beta1 || b2 != s->beta2) {
        s->step = step;
        s->beta1 = b1;
        s->beta2 = b2;
        s->beta1_t = (float)pow((double)b1, (double)step);
        s->beta2_t = (float)pow((double)b2, (double)step);
        return;
    }
    s->step += 1;
    if (s->step != step) {
        s->beta1_t = (float)pow((double)s->beta1, (double)step);
        s->beta2_t = (float)pow((double)s->beta2, (double)step);
        s->step = step;
    } else {
        s->beta1_t = s->beta1_t * s->beta1;
        s->beta2_t = s->beta2_t * s->beta2;
    }
}

static void update_state(oracle_adam* s, float lr, float eps, float wd, int bias_correction) {
    s->alpha = lr;
    s->eps = eps;
    s->weight_decay = wd;
    s->bc1 = 1.0f;
    s->bc2 = 1.0f;
    if (bias_correction) {
        s->bc1 = 1.0f - s->beta1_t;
        s->bc2 = 1.0f / sqrtf(1.0f - s->beta2_t);
    }
}

/* Scalars of the current call, exposed for tests. */
void oracle_adam_scalars(const oracle_adam* s, float* bc1, float* bc2) {
    *bc1 = s->bc1;
    *bc2 = s->bc2;
}

void oracle_adam_update(oracle_adam* s, size_t step, float lr, float b1, float b2, float eps,
                        float wd, int bias_correction, float* p, const float* g, float* m,
                        float* v, size_t n) {
    increment_step(s, step, b1, b2);
    update_state(s, lr, eps, wd, bias_correction);
    const float beta1 = s->beta1, beta2 = s->beta2;
    const float b1m1 = 1.0f - beta1, b2m1 = 1.0f - beta2;
    const float step_size = -1.0f * s->alpha / s->bc1;
    const float w_decay = -1.0f * s->alpha * s->weight_decay;
    const int decay = s->weight_decay > 0.0f;
    const size_t n_main = n - n % 16;
    for (size_t i = 0; i < n; ++i) {
        float gi = g[i], pi = p[i], mi = m[i], vi = v[i];
        if (decay && !s->adamw_mode) gi = fmaf(pi, s->weight_decay, gi);
        if (i < n_main) {
            mi = mi * beta1;
            mi = fmaf(gi, b1m1, mi);
            vi = vi * beta2;
            gi = gi * gi;
            vi = fmaf(gi, b2m1, vi);
        } else {
            const float gb = gi * b1m1;
            mi = fmaf(mi, beta1, gb);
            gi = gi * gi;
            const float gv = gi * b2m1;
            vi = fmaf(vi, beta2, gv);
        }
        float d = fmaf(sqrtf(vi), s->bc2, s->eps);
        d = mi / d;
        if (decay && s->adamw_mode) pi = fmaf(pi, w_decay, pi);
        pi = fmaf(d, step_size, pi);
        p[i] = pi;
        m[i] = mi;
        v[i] = vi;
    }
}
