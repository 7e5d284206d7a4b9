/* Exhaustive check of the activation quantizer's fast quotient.
 *
 * For 16-bit activations (fp16 or bf16) and a finite normal row scale s, the A8 prologue computes
 * x / s as q = fma(fma(-x*y, s, x), y, x*y) with y = RN(1/s) (one Markstein residual correction)
 * instead of the IEEE division, then quantizes t = clamp(rint(round16(q)), -128, 127).
 *
 * This program walks every scale s of the 16-bit format that takes the fast path and every
 * finite 16-bit x with |x| <= 130 s (the quantizer's domain: |x| <= absmax <= 127.06 s) and counts
 *   - fp32 quotients that differ from IEEE x / s (ignoring the sign of a zero quotient), and
 *   - int8 results that differ.
 * It prints "<fmt> pairs=N f32_mismatch=A int8_mismatch=B".
 *
 * Build: gcc -O2 -ffp-contract=off quotient_check.c -lm -lpthread; run with "h" (fp16) or "b" (bf16).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static int g_bf;

static float f16_to_f32(uint16_t h) {
    const uint32_t sg = (h >> 15) & 1, e = (h >> 10) & 31, m = h & 1023;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(m | 1024), (int)e - 25);
    return sg ? -v : v;
}
static float bf16_to_f32(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static uint32_t bits_of(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static float to_f32(int code) { return g_bf ? bf16_to_f32((uint16_t)code) : f16_to_f32((uint16_t)code); }

/* round-to-nearest-even to the 16-bit format and back (finite |f| well inside the range) */
static float round16(float f) {
    if (f == 0 || isnan(f)) return f;
    if (g_bf) {
        uint32_t u = bits_of(f);
        u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
        float r;
        memcpy(&r, &u, 4);
        return r;
    }
    const float a = fabsf(f);
    if (a < 0x1p-14f) return rintf(f * 0x1p24f) * 0x1p-24f; /* fp16 subnormal grid */
    int e;
    frexpf(a, &e);
    const float sc = ldexpf(1.0f, e - 11);
    const float r = rintf(f / sc) * sc;
    return fabsf(r) > 65504.0f ? copysignf(INFINITY, f) : r;
}
static float quant(float q) { return fminf(fmaxf(rintf(round16(q)), -128.0f), 127.0f); }

typedef struct {
    int lo, hi;
    long long pairs, f32_bad, int8_bad;
} job_t;

static void* run(void* arg) {
    job_t* j = (job_t*)arg;
    for (int sc = j->lo; sc < j->hi; ++sc) {
        const float s = to_f32(sc);
        if (!(s >= 0x1p-126f) || isinf(s)) continue; /* the kernel's fast-path condition */
        const float y = 1.0f / s;
        for (int xc = 0; xc < 65536; ++xc) {
            const float x = to_f32(xc);
            /* an infinite element makes the row scale infinite, which takes the IEEE path */
            if (!isfinite(x) || fabsf(x) > 130.0f * s) continue;
            const float ref = x / s;
            const float q0 = x * y;
            const float q = fmaf(fmaf(-q0, s, x), y, q0);
            j->pairs++;
            if (bits_of(q) != bits_of(ref) && !(q == 0 && ref == 0)) j->f32_bad++;
            if (quant(q) != quant(ref)) j->int8_bad++;
        }
    }
    return 0;
}

int main(int argc, char** argv) {
    g_bf = argc > 1 && argv[1][0] == 'b';
    enum { T = 8 };
    pthread_t th[T];
    job_t jobs[T];
    for (int t = 0; t < T; ++t) {
        jobs[t] = (job_t){1 + t * (0x7fff / T), t == T - 1 ? 0x7fff : 1 + (t + 1) * (0x7fff / T), 0, 0, 0};
        pthread_create(&th[t], 0, run, &jobs[t]);
    }
    long long pairs = 0, fb = 0, ib = 0;
    for (int t = 0; t < T; ++t) {
        pthread_join(th[t], 0);
        pairs += jobs[t].pairs;
        fb += jobs[t].f32_bad;
        ib += jobs[t].int8_bad;
    }
    printf("%s pairs=%lld f32_mismatch=%lld int8_mismatch=%lld\n", g_bf ? "bf16" : "fp16", pairs, fb, ib);
    return 0;
}
