/* The A8 weight decoders' int8 grid value against the reference's definition
 * (roblennon/mac-kernels-public modal/weight_error_app.py:335-337):
 *     w8 = clamp(rne(fp32(level * s)), -127, 127)
 * The kernels compute it as
 *     v = level * s                       (one fp32 product: codebook levels, the 4-bit tables and
 *                                          the per-code decoder)
 *     v = fma(c, s', -2^(bits-1) s')      (the 6-bit decoder's uniform levels c - 2^(bits-1); the
 *                                          exact product rounded once, s' = s clamped to +-2^20)
 *     t = med3(v + 1.5 * 2^23, M - 127, M + 127)       (the add rounds to an integer, ties to even)
 *     w8 = low byte of bits(t)
 * Checked, both forms for uniform levels: every 4- and 6-bit code against every finite fp16, bf16
 * and e4m3 scale; 2^24 random fp32 scales spread over every exponent; and the fixed 16-level
 * codebook against every fp16, bf16 and e4m3 scale.  Prints "checked=N mismatch=M".  CPU only (gcc -ffp-contract=off). */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float h2f(uint16_t h) {
    uint32_t s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
    float v = e == 0 ? ldexpf((float)m, -24) : e == 31 ? (m ? NAN : INFINITY) : ldexpf((float)(m | 1024), (int)e - 25);
    return s ? -v : v;
}
static float e4m3(uint8_t b) {
    uint32_t s = b >> 7, e = (b >> 3) & 15, m = b & 7;
    if (e == 15 && m == 7) return NAN;
    float v = e ? ldexpf((float)(8 | m), (int)e - 10) : ldexpf((float)m, -9);
    return s ? -v : v;
}
static const float CB[16] = {-0.980602f, -0.794529f, -0.638165f, -0.500986f, -0.377321f, -0.263187f, -0.155210f,
                             -0.050720f, 0.052541f,  0.156985f,  0.265284f,  0.379533f,  0.502636f,  0.638953f,
                             0.794876f,  0.980671f};
static long checked = 0, mismatch = 0;
static const float MAGIC = 12582912.0f;

static int8_t reference(float level, float s) {
    float p = level * s;  /* one fp32 product */
    float r = rintf(p);
    if (r < -127.0f) r = -127.0f;
    if (r > 127.0f) r = 127.0f;
    return (int8_t)(int)r;
}
static int8_t med3_byte(float v) {
    float t = v + MAGIC;
    if (!(t >= MAGIC - 127.0f)) t = MAGIC - 127.0f;  /* med3(t, lo, hi) for t finite or infinite */
    if (t > MAGIC + 127.0f) t = MAGIC + 127.0f;
    return (int8_t)(f2u(t) & 0xFFu);
}
static void uniform(float s, int bits) {
    if (!isfinite(s)) return;
    const int half = 1 << (bits - 1);
    const float sc = fminf(fmaxf(s, -1048576.0f), 1048576.0f);
    const float off = -(float)half * sc;
    for (int c = 0; c < (1 << bits); ++c) {
        const int8_t want = reference((float)(c - half), s);
        const int8_t got_fma = med3_byte(fmaf((float)c, sc, off)), got_mul = med3_byte((float)(c - half) * s);
        checked += 2;
        if (got_fma != want && mismatch++ < 5) printf("uniform fma bits=%d c=%d s=%a: want %d got %d\n", bits, c, s, want, got_fma);
        if (got_mul != want && mismatch++ < 5) printf("uniform mul bits=%d c=%d s=%a: want %d got %d\n", bits, c, s, want, got_mul);
    }
}
static void codebook(float s) {
    if (!isfinite(s)) return;
    for (int c = 0; c < 16; ++c) {
        int8_t want = reference(CB[c], s), got = med3_byte(CB[c] * s);
        ++checked;
        if (got != want && mismatch++ < 5) printf("codebook c=%d s=%a: want %d got %d\n", c, s, want, got);
    }
}
int main(void) {
    for (uint32_t h = 0; h < 65536; ++h) { uniform(h2f((uint16_t)h), 4); uniform(h2f((uint16_t)h), 6); codebook(h2f((uint16_t)h)); }
    for (uint32_t b = 0; b < 65536; ++b) { uniform(u2f(b << 16), 4); uniform(u2f(b << 16), 6); codebook(u2f(b << 16)); }
    for (uint32_t b = 0; b < 256; ++b) { uniform(e4m3((uint8_t)b), 4); uniform(e4m3((uint8_t)b), 6); codebook(e4m3((uint8_t)b)); }
    uint64_t x = 0x9E3779B97F4A7C15ull;  /* xorshift: fp32 scales with every exponent */
    for (int i = 0; i < (1 << 24); ++i) {
        x ^= x << 13; x ^= x >> 7; x ^= x << 17;
        const uint32_t u = (uint32_t)x;
        uniform(u2f(u), 6);
        if ((i & 7) == 0) { uniform(u2f(u), 4); codebook(u2f(u)); }
    }
    printf("checked=%ld mismatch=%ld\n", checked, mismatch);
    return mismatch != 0;
}
