/*
 * CPU oracle for the quantized-linear path. TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C, the arithmetic of the reference's packed-weight codecs so
 * that the HIP product path can be checked against it.  Only tests/, the smoke check and the
 * CPU-baseline leg of bench.py may load it; the product library never links or calls it.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fno-fast-math).  Contraction must stay off:
 * the reference computes every decode with separately rounded fp32 multiplies and adds.
 *
 * Sources followed (reference repository, roblennon/mac-kernels-public):
 *   GGUF block layouts and per-type formulas ........ docs/research/2026-10-03-gguf-on-metal.md:18-36
 *   Q8_0 / Q4_0 closed forms ......................... modal/modal_app.py:32-50
 *   gguf-py 0.19.0 dequantize (third-party, named at modal/weight_error_app.py:55 and called at
 *     bench/bench_gguf_linear.py:92): operation order restated per type below.
 *   INT8 rowwise quantize / dequantize .............. modal/weight_error_app.py:109-127
 *   Hadamard construction ............................ modal/weight_error_app.py:90-98
 *   W4A8/W6A8 unpack and int8-grid decode ............ modal/weight_error_app.py:155-166, 326-339
 *
 * Parity status per function is recorded in the header comment of each function.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#if defined(__FP_FAST_FMA) || defined(__FAST_MATH__)
#error "the oracle must be compiled without fast-math"
#endif

/* ------------------------------------------------------------------------------------------
 * Scalar format conversions (exact, by bit manipulation).
 * ---------------------------------------------------------------------------------------- */

static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* IEEE binary16 -> binary32, exact for every input (subnormals, inf, NaN payload kept). */
float qlo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    if (exp == 0x1Fu) return bits_f32(sign | 0x7F800000u | (man << 13));
    if (exp != 0) return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
    if (man == 0) return bits_f32(sign);
    /* subnormal: value = man * 2^-24, representable exactly in fp32 */
    float v = (float)man * bits_f32(0x33800000u); /* 2^-24 */
    return (sign ? -v : v);
}

/* binary32 -> binary16, round to nearest even, overflow to inf (the behaviour of a float->half
 * cast in torch and of the hardware conversion). */
uint16_t qlo_f32_to_f16(float f) {
    uint32_t u = f32_bits(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x3FFu)); /* NaN */
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to inf */
    if (a < 0x38800000u) {
        /* result is subnormal or zero: quantum 2^-24.  a < 2^-14. */
        if (a < 0x33000000u) return sign; /* < 2^-25: rounds to zero (2^-25 ties to even 0) */
        uint32_t e = a >> 23;            /* biased exponent, 102..112 */
        uint32_t m = (a & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e;       /* value = m * 2^(e-150); quantum 2^-24 -> shift by (126-e) */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    /* normal range */
    uint32_t e = (a >> 23) - 112u;
    uint32_t m = a & 0x7FFFFFu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

float qlo_bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

/* float8_e4m3fn -> fp32 (bias 7, no infinities, S.1111.111 is NaN). */
float qlo_e4m3_to_f32(uint8_t v) {
    uint32_t sign = (uint32_t)(v & 0x80u) << 24;
    uint32_t exp = (v >> 3) & 0xFu;
    uint32_t man = v & 0x7u;
    if (exp == 0xFu && man == 0x7u) return bits_f32(sign | 0x7FC00000u);
    if (exp == 0) {
        float x = (float)man * 0.001953125f; /* man * 2^-9 */
        return sign ? -x : x;
    }
    return bits_f32(sign | ((exp + 120u) << 23) | (man << 20));
}

/* fp32 -> float8_e4m3fn, round to nearest even.  A magnitude that rounds to the bit pattern
 * above 448 (S.1111.111) is NaN, and so is anything >= 480, as torch's float8_e4m3fn cast
 * behaves; 464 (the midpoint of 448 and 480) ties to the even 448. */
uint8_t qlo_f32_to_e4m3(float f) {
    uint32_t u = f32_bits(f);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    float a = fabsf(f);
    if (isnan(f) || a >= 480.0f) return (uint8_t)(sign | 0x7Fu);
    if (a < 0.015625f) {
        /* subnormal grid 2^-9 */
        double q = nearbyint((double)a * 512.0); /* exact scaling; default rounding is to even */
        return (uint8_t)(sign | (uint8_t)q);   /* q==8 gives 0x08 = 2^-6, the smallest normal */
    }
    int e;
    double m = frexp((double)a, &e); /* a = m * 2^e, m in [0.5,1) */
    double scaled = ldexp(m, 4);     /* 8..16: keep 3 fraction bits */
    double q = nearbyint(scaled);    /* 8..16 */
    if (q >= 16.0) { q = 8.0; e += 1; }
    int biased = e - 1 + 7;
    uint8_t out = (uint8_t)(((unsigned)biased << 3) | ((unsigned)q - 8u));
    if (out > 0x7Eu) out = 0x7Fu;
    return (uint8_t)(sign | out);
}

/* ------------------------------------------------------------------------------------------
 * GGUF block decode.  Each function decodes ONE block into fp32 exactly as gguf-py 0.19.0
 * computes it (fp32, separately rounded operations).  Layouts: gguf-on-metal.md:18-36.
 * ---------------------------------------------------------------------------------------- */

static inline float rd_f16(const uint8_t* p) { return qlo_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* Q4_0: f16 d, qs[16]; value j<16 = d*(lo(qs[j])-8), j>=16 = d*(hi(qs[j-16])-8).
 * Pinned by the closed form at modal/modal_app.py:42-50 (tests brute-force it). */
static void dq_q4_0(const uint8_t* b, float* y) {
    float d = rd_f16(b);
    for (int j = 0; j < 16; ++j) {
        y[j] = d * (float)((int)(b[2 + j] & 0xF) - 8);
        y[j + 16] = d * (float)((int)(b[2 + j] >> 4) - 8);
    }
}

/* Q4_1: f16 d, f16 m, qs[16]; value = d*nib + m (gguf-on-metal.md:21). */
static void dq_q4_1(const uint8_t* b, float* y) {
    float d = rd_f16(b), m = rd_f16(b + 2);
    for (int j = 0; j < 16; ++j) {
        float lo = d * (float)(b[4 + j] & 0xF);
        float hi = d * (float)(b[4 + j] >> 4);
        y[j] = lo + m;
        y[j + 16] = hi + m;
    }
}

/* Q5_0: f16 d, u32 qh (little endian), qs[16]; value j = d*((nib | bit j of qh << 4) - 16). */
static void dq_q5_0(const uint8_t* b, float* y) {
    float d = rd_f16(b);
    uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
    for (int j = 0; j < 16; ++j) {
        int lo = (b[6 + j] & 0xF) | (int)(((qh >> j) & 1u) << 4);
        int hi = (b[6 + j] >> 4) | (int)(((qh >> (j + 16)) & 1u) << 4);
        y[j] = d * (float)(lo - 16);
        y[j + 16] = d * (float)(hi - 16);
    }
}

/* Q5_1: f16 d, f16 m, u32 qh, qs[16]; value = d*q + m. */
static void dq_q5_1(const uint8_t* b, float* y) {
    float d = rd_f16(b), m = rd_f16(b + 2);
    uint32_t qh = (uint32_t)b[4] | ((uint32_t)b[5] << 8) | ((uint32_t)b[6] << 16) | ((uint32_t)b[7] << 24);
    for (int j = 0; j < 16; ++j) {
        int lo = (b[8 + j] & 0xF) | (int)(((qh >> j) & 1u) << 4);
        int hi = (b[8 + j] >> 4) | (int)(((qh >> (j + 16)) & 1u) << 4);
        float a0 = d * (float)lo, a1 = d * (float)hi;
        y[j] = a0 + m;
        y[j + 16] = a1 + m;
    }
}

/* Q8_0: f16 d, i8 qs[32]; value = qs[j]*d (modal/modal_app.py:32-39). Pinned by golden vectors. */
static void dq_q8_0(const uint8_t* b, float* y) {
    float d = rd_f16(b);
    for (int j = 0; j < 32; ++j) y[j] = (float)(int8_t)b[2 + j] * d;
}

/* Q2_K: scales[16], qs[64], f16 d @80, f16 dmin @82.  Per 16 values s:
 *   dl = d*(sc&15), ml = dmin*(sc>>4), value = dl*q - ml, q = (qs[32h+i] >> 2t) & 3
 * where v = 128h + 32t + i (gguf-on-metal.md:25). */
static void dq_q2_k(const uint8_t* b, float* y) {
    float d = rd_f16(b + 80), dmin = rd_f16(b + 82);
    for (int v = 0; v < 256; ++v) {
        int s = v >> 4;
        float dl = d * (float)(b[s] & 0xF);
        float ml = dmin * (float)(b[s] >> 4);
        int h = v >> 7, t = (v >> 5) & 3, i = v & 31;
        int q = (b[16 + 32 * h + i] >> (2 * t)) & 3;
        float p = dl * (float)q;
        y[v] = p - ml;
    }
}

/* Q3_K: hmask[32], qs[64], scales[12], f16 d @108.  16 signed 6-bit scales:
 *   low 4 bits = scales[s%8] >> 4*(s/8), high 2 bits = scales[8 + s%4] >> 2*(s/4), minus 32.
 * value v (h = v/128, t = (v%128)/32, i = v%32):
 *   q2 = (qs[32h+i] >> 2t) & 3, hbit = (hmask[i] >> (v/32)) & 1, q = q2 - 4*(1-hbit)
 *   value = (d*s6) * q  (gguf-on-metal.md:26, 36). */
static void dq_q3_k(const uint8_t* b, float* y) {
    const uint8_t* hm = b;
    const uint8_t* qs = b + 32;
    const uint8_t* sc = b + 96;
    float d = rd_f16(b + 108);
    for (int v = 0; v < 256; ++v) {
        int s = v >> 4;
        int lo = (sc[s & 7] >> (4 * (s >> 3))) & 0xF;
        int hi = (sc[8 + (s & 3)] >> (2 * (s >> 2))) & 3;
        int s6 = (lo | (hi << 4)) - 32;
        float dl = d * (float)s6;
        int h = v >> 7, t = (v >> 5) & 3, i = v & 31;
        int q2 = (qs[32 * h + i] >> (2 * t)) & 3;
        int hb = (hm[i] >> (v >> 5)) & 1;
        int q = q2 - ((hb ^ 1) << 2);
        y[v] = dl * (float)q;
    }
}

/* Q4_K/Q5_K 12-byte scale packing (gguf-on-metal.md:33). */
static void kquant_scale_min(const uint8_t* s, int j, int* sc, int* mn) {
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* Q4_K: f16 d, f16 dmin, scales[12], qs[128].  Sub-block j (32 values) lives in chunk c=j/2
 * (qs[32c..32c+32)), low nibbles for even j, high for odd.  value = (d*sc)*q - dmin*m.
 * Pinned by golden vectors (gguf_q4_k). */
static void dq_q4_k(const uint8_t* b, float* y) {
    float d = rd_f16(b), dmin = rd_f16(b + 2);
    const uint8_t* qs = b + 16;
    for (int j = 0; j < 8; ++j) {
        int sc, mn;
        kquant_scale_min(b + 4, j, &sc, &mn);
        float dl = d * (float)sc;
        float ml = dmin * (float)mn;
        int c = j >> 1, sh = (j & 1) * 4;
        for (int i = 0; i < 32; ++i) {
            int q = (qs[32 * c + i] >> sh) & 0xF;
            float p = dl * (float)q;
            y[32 * j + i] = p - ml;
        }
    }
}

/* Q5_K: f16 d, f16 dmin, scales[12], qh[32], qs[128]; fifth bit of value i of sub-block j is
 * bit j of qh[i] (gguf-on-metal.md:28, 34). */
static void dq_q5_k(const uint8_t* b, float* y) {
    float d = rd_f16(b), dmin = rd_f16(b + 2);
    const uint8_t* qh = b + 16;
    const uint8_t* qs = b + 48;
    for (int j = 0; j < 8; ++j) {
        int sc, mn;
        kquant_scale_min(b + 4, j, &sc, &mn);
        float dl = d * (float)sc;
        float ml = dmin * (float)mn;
        int c = j >> 1, sh = (j & 1) * 4;
        for (int i = 0; i < 32; ++i) {
            int q = ((qs[32 * c + i] >> sh) & 0xF) | (((qh[i] >> j) & 1) << 4);
            float p = dl * (float)q;
            y[32 * j + i] = p - ml;
        }
    }
}

/* Q6_K: ql[128], qh[64], i8 scales[16], f16 d @208.  value v (h = v/128, r = v%128):
 *   lo = (ql[64h + r%64] >> 4*(r/64)) & 15, hi = (qh[32h + r%32] >> 2*(r/32)) & 3,
 *   q = (lo | hi<<4) - 32, value = (d*scales[v/16]) * q  (gguf-on-metal.md:29, 35). */
static void dq_q6_k(const uint8_t* b, float* y) {
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const int8_t* sc = (const int8_t*)(b + 192);
    float d = rd_f16(b + 208);
    for (int v = 0; v < 256; ++v) {
        int h = v >> 7, r = v & 127;
        int lo = (ql[64 * h + (r & 63)] >> (4 * (r >> 6))) & 0xF;
        int hi = (qh[32 * h + (r & 31)] >> (2 * (r >> 5))) & 3;
        int q = (lo | (hi << 4)) - 32;
        float dl = d * (float)sc[v >> 4];
        y[v] = dl * (float)q;
    }
}

/* IQ4_NL / IQ4_XS non-linear levels.  Not in the reference repository; this is ggml's public
 * 16-entry table (ggml-common.h kvalues_iq4nl, MIT), used by gguf-py 0.19.0's IQ4_NL/IQ4_XS
 * dequantize.  Parity unpinned by reference vectors (see the tests for the invariants used). */
static const int8_t kIQ4NL[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

/* IQ4_NL: f16 d, qs[16]; value j<16 = d*K[lo(qs[j])], j>=16 = d*K[hi(qs[j-16])]. */
static void dq_iq4_nl(const uint8_t* b, float* y) {
    float d = rd_f16(b);
    for (int j = 0; j < 16; ++j) {
        y[j] = d * (float)kIQ4NL[b[2 + j] & 0xF];
        y[j + 16] = d * (float)kIQ4NL[b[2 + j] >> 4];
    }
}

/* IQ4_XS: f16 d @0, u16 scales_h @2, u8 scales_l[4] @4, qs[128] @8.  Sub-block s (32 values):
 *   ls = ((scales_l[s/2] >> 4*(s%2)) & 15) | (((scales_h >> 2s) & 3) << 4), dl = d*(ls-32),
 *   value i<16 = dl*K[lo(qs[16s+i])], i>=16 = dl*K[hi(qs[16s+i-16])]. */
static void dq_iq4_xs(const uint8_t* b, float* y) {
    float d = rd_f16(b);
    uint32_t sh = (uint32_t)b[2] | ((uint32_t)b[3] << 8);
    for (int s = 0; s < 8; ++s) {
        int ls = ((b[4 + (s >> 1)] >> (4 * (s & 1))) & 0xF) | (int)(((sh >> (2 * s)) & 3u) << 4);
        float dl = d * (float)(ls - 32);
        const uint8_t* qs = b + 8 + 16 * s;
        for (int i = 0; i < 16; ++i) {
            y[32 * s + i] = dl * (float)kIQ4NL[qs[i] & 0xF];
            y[32 * s + 16 + i] = dl * (float)kIQ4NL[qs[i] >> 4];
        }
    }
}

typedef void (*dq_fn)(const uint8_t*, float*);

/* ggml type id -> (values per block, bytes per block, decoder).  Ids follow enum ggml_type
 * (Q8_0 = 8 and Q4_K = 12 are pinned at modal/weight_error_app.py:84). */
static int gguf_info(int type, int* qk, int* ts, dq_fn* fn) {
    switch (type) {
        case 2:  *qk = 32;  *ts = 18;  *fn = dq_q4_0;  return 0;
        case 3:  *qk = 32;  *ts = 20;  *fn = dq_q4_1;  return 0;
        case 6:  *qk = 32;  *ts = 22;  *fn = dq_q5_0;  return 0;
        case 7:  *qk = 32;  *ts = 24;  *fn = dq_q5_1;  return 0;
        case 8:  *qk = 32;  *ts = 34;  *fn = dq_q8_0;  return 0;
        case 10: *qk = 256; *ts = 84;  *fn = dq_q2_k;  return 0;
        case 11: *qk = 256; *ts = 110; *fn = dq_q3_k;  return 0;
        case 12: *qk = 256; *ts = 144; *fn = dq_q4_k;  return 0;
        case 13: *qk = 256; *ts = 176; *fn = dq_q5_k;  return 0;
        case 14: *qk = 256; *ts = 210; *fn = dq_q6_k;  return 0;
        case 20: *qk = 32;  *ts = 18;  *fn = dq_iq4_nl; return 0;
        case 23: *qk = 256; *ts = 136; *fn = dq_iq4_xs; return 0;
        default: return -1;
    }
}

int qlo_gguf_block_info(int type, int* qk, int* ts) {
    dq_fn fn;
    return gguf_info(type, qk, ts, &fn);
}

/* Decode `nblocks` consecutive blocks of `type` from `src` into `dst` (nblocks*qk floats). */
int qlo_gguf_dequantize(int type, const uint8_t* src, int64_t nblocks, float* dst) {
    int qk, ts;
    dq_fn fn;
    if (gguf_info(type, &qk, &ts, &fn)) return -1;
    for (int64_t i = 0; i < nblocks; ++i) fn(src + i * ts, dst + i * qk);
    return 0;
}

/* Decode a flat element range [e0, e0+count) of a tensor stored as consecutive blocks,
 * indexing by flat element (block = e/qk), which also covers rows that straddle blocks
 * (gguf-on-metal.md:38). */
int qlo_gguf_dequantize_range(int type, const uint8_t* src, int64_t e0, int64_t count, float* dst) {
    int qk, ts;
    dq_fn fn;
    if (gguf_info(type, &qk, &ts, &fn)) return -1;
    float tmp[256];
    int64_t e = e0, end = e0 + count;
    while (e < end) {
        int64_t blk = e / qk;
        fn(src + blk * ts, tmp);
        int64_t off = e - blk * qk;
        int64_t take = qk - off;
        if (take > end - e) take = end - e;
        memcpy(dst + (e - e0), tmp + off, (size_t)take * sizeof(float));
        e += take;
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------
 * INT8 rowwise (modal/weight_error_app.py:109-127).
 * ---------------------------------------------------------------------------------------- */

/* Decode: out[n,k] = float(q[n,k]) * scale[n] (weight_error_app.py:122-123). Pinned by the
 * golden int8_rowwise deq sha256. */
void qlo_dequantize_int8(const int8_t* q, const float* scale, int64_t n, int64_t k, float* out) {
    for (int64_t r = 0; r < n; ++r) {
        float s = scale[r];
        for (int64_t c = 0; c < k; ++c) out[r * k + c] = (float)q[r * k + c] * s;
    }
}

/* Round half to even on a float that is already a small integer-or-tie candidate. */
static inline float rne(float v) { return nearbyintf(v); }

/* quantize_int8_rowwise on fp32 rows (weight_error_app.py:109-115), x.dtype = float32:
 *   scale = max(absmax/127, 1e-30) (fp32); s = scale (same dtype), zero -> FLT_MIN;
 *   q = clamp(rne(x / s), -128, 127).
 * Pinned by the golden int8_rowwise q/scale sha256. */
void qlo_quantize_int8_rowwise_f32(const float* x, int64_t m, int64_t k, int8_t* q, float* scale) {
    for (int64_t r = 0; r < m; ++r) {
        const float* row = x + r * k;
        float amax = 0.0f;
        for (int64_t c = 0; c < k; ++c) { float a = fabsf(row[c]); if (a > amax) amax = a; }
        float s = amax / 127.0f;
        if (s < 1e-30f) s = 1e-30f;
        scale[r] = s;
        float sd = s; /* .to(float32) is the identity; s is never zero after the clamp */
        if (sd == 0.0f) sd = 1.17549435e-38f;
        for (int64_t c = 0; c < k; ++c) {
            float v = rne(row[c] / sd);
            if (v < -128.0f) v = -128.0f;
            if (v > 127.0f) v = 127.0f;
            q[r * k + c] = (int8_t)v;
        }
    }
}

/* quantize_int8_rowwise on fp16 rows (the A8 activation quantization, weight_error_app.py:109-115
 * with x.dtype = float16):
 *   scale = max(float(absmax)/127, 1e-30) in fp32; s = fp16(scale), zero -> fp16 tiny (2^-14);
 *   q = clamp(rne(fp16(float(x)/float(s))), -128, 127)  (torch computes the fp16 division in
 *   fp32 and rounds the quotient to fp16 before round()).
 * Inputs/outputs are raw fp16 bit patterns. */
void qlo_quantize_int8_rowwise_f16(const uint16_t* x, int64_t m, int64_t k, int8_t* q, float* scale) {
    for (int64_t r = 0; r < m; ++r) {
        const uint16_t* row = x + r * k;
        float amax = 0.0f;
        for (int64_t c = 0; c < k; ++c) { float a = fabsf(qlo_f16_to_f32(row[c])); if (a > amax || isnan(a)) amax = a; }
        float s = amax / 127.0f;
        if (s < 1e-30f) s = 1e-30f;
        scale[r] = s;
        float s16 = qlo_f16_to_f32(qlo_f32_to_f16(s));
        if (s16 == 0.0f) s16 = 6.103515625e-05f; /* torch.finfo(float16).tiny = 2^-14 */
        for (int64_t c = 0; c < k; ++c) {
            float quot = qlo_f16_to_f32(qlo_f32_to_f16(qlo_f16_to_f32(row[c]) / s16));
            float v = rne(quot);
            if (v < -128.0f) v = -128.0f;
            if (v > 127.0f) v = 127.0f;
            q[r * k + c] = (int8_t)v;
        }
    }
}

/* bf16 rounding (round to nearest even), as a float. */
static float round_bf16(float f) {
    uint32_t u = f32_bits(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return f;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return bits_f32(u & 0xFFFF0000u);
}

/* quantize_int8_rowwise on bf16 rows (x.dtype = bfloat16): as the fp16 version with bf16
 * rounding of the scale and of the quotient; zero scale -> finfo(bfloat16).tiny = 2^-126.
 * Inputs are raw bf16 bit patterns. */
void qlo_quantize_int8_rowwise_bf16(const uint16_t* x, int64_t m, int64_t k, int8_t* q, float* scale) {
    for (int64_t r = 0; r < m; ++r) {
        const uint16_t* row = x + r * k;
        float amax = 0.0f;
        for (int64_t c = 0; c < k; ++c) { float a = fabsf(qlo_bf16_to_f32(row[c])); if (a > amax || isnan(a)) amax = a; }
        float s = amax / 127.0f;
        if (s < 1e-30f) s = 1e-30f;
        scale[r] = s;
        float sb = round_bf16(s);
        if (sb == 0.0f) sb = 1.17549435e-38f;
        for (int64_t c = 0; c < k; ++c) {
            float v = rne(round_bf16(qlo_bf16_to_f32(row[c]) / sb));
            if (v < -128.0f) v = -128.0f;
            if (v > 127.0f) v = 127.0f;
            q[r * k + c] = (int8_t)v;
        }
    }
}

/* ------------------------------------------------------------------------------------------
 * Hadamard rotation.
 * ---------------------------------------------------------------------------------------- */

/* Unnormalized +-1 Hadamard entry for size G.  For G a power of 4 this is the Kronecker power
 * of H4 = [[1,1,1,-1],[1,1,-1,1],[1,-1,1,1],[-1,1,1,1]] (weight_error_app.py:90-98), with the
 * first factor most significant (torch.kron(h, h4) appends h4 as the least significant digit).
 * H4[i][j] = -1 iff i + j == 3.  For G = 2*4^p (not a power of 4) the construction is
 * H2 (x) H4^(x)p with H2 = [[1,1],[1,-1]] as the most significant factor; this size has no
 * counterpart in the reference (parity unpinned, checked through its invariants). */
int qlo_hadamard_sign(int g, int i, int j) {
    int sgn = 1;
    int rest = g;
    /* least significant radix-4 digits first */
    while (rest >= 4) {
        int di = i & 3, dj = j & 3;
        if (di + dj == 3) sgn = -sgn;
        i >>= 2; j >>= 2; rest >>= 2;
    }
    if (rest == 2) {
        if ((i & 1) && (j & 1)) sgn = -sgn;
    }
    return sgn;
}

static int valid_group(int g) {
    if (g < 2) return 0;
    int x = g;
    while (x >= 4 && (x & 3) == 0) x >>= 2;
    return x == 1 || x == 2;
}

int qlo_hadamard_valid(int g) { return valid_group(g); }

/* Exact rotation of fp32 rows: out[:, grp] = in[:, grp] @ H^T with H normalized by 1/sqrt(G).
 * Sums are taken in long double/double by the fast Walsh-Hadamard butterflies (exact for the
 * fp16/bf16-valued inputs this path sees: their 256 partial sums fit in 53 bits), then scaled
 * by 1/sqrt(G) and rounded once to fp32.  For G = 4^p the scale 2^-p is exact.  H is symmetric
 * so x @ H^T == x @ H.  The reference rotates through BLAS (weight_error_app.py:101-106), whose
 * summation order is platform-dependent; this restatement is the correctly rounded value. */
int qlo_rotate_f32(const float* in, int64_t rows, int64_t k, int g, float* out) {
    if (!valid_group(g) || k % g) return -1;
    double* buf = (double*)malloc(sizeof(double) * (size_t)g);
    double inv = 1.0 / sqrt((double)g);
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t c0 = 0; c0 < k; c0 += g) {
            for (int j = 0; j < g; ++j) buf[j] = (double)in[r * k + c0 + j];
            /* radix-4 stages on the least significant digits, then an optional radix-2 stage */
            int stride = 1;
            int rest = g;
            while (rest >= 4) {
                for (int base = 0; base < g; base += 4 * stride) {
                    for (int o = 0; o < stride; ++o) {
                        double a0 = buf[base + o], a1 = buf[base + o + stride];
                        double a2 = buf[base + o + 2 * stride], a3 = buf[base + o + 3 * stride];
                        /* y_i = sum_j H4[i][j] a_j = S - 2*a_{3-i} */
                        double s = a0 + a1 + a2 + a3;
                        buf[base + o] = s - 2.0 * a3;
                        buf[base + o + stride] = s - 2.0 * a2;
                        buf[base + o + 2 * stride] = s - 2.0 * a1;
                        buf[base + o + 3 * stride] = s - 2.0 * a0;
                    }
                }
                stride *= 4;
                rest >>= 2;
            }
            if (rest == 2) {
                for (int o = 0; o < stride; ++o) {
                    double a0 = buf[o], a1 = buf[o + stride];
                    buf[o] = a0 + a1;
                    buf[o + stride] = a0 - a1;
                }
            }
            for (int j = 0; j < g; ++j) out[r * k + c0 + j] = (float)(buf[j] * inv);
        }
    }
    free(buf);
    return 0;
}

/* Rotation of fp16 activations followed by one rounding to fp16 (the weight-only and A8
 * prologues compute the rotation exactly and round once). */
int qlo_rotate_f16(const uint16_t* in, int64_t rows, int64_t k, int g, uint16_t* out) {
    if (!valid_group(g) || k % g) return -1;
    float* tmp_in = (float*)malloc(sizeof(float) * (size_t)k);
    float* tmp_out = (float*)malloc(sizeof(float) * (size_t)k);
    double* buf = (double*)malloc(sizeof(double) * (size_t)g);
    double inv = 1.0 / sqrt((double)g);
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t c = 0; c < k; ++c) tmp_in[c] = qlo_f16_to_f32(in[r * k + c]);
        for (int64_t c0 = 0; c0 < k; c0 += g) {
            for (int j = 0; j < g; ++j) buf[j] = (double)tmp_in[c0 + j];
            int stride = 1, rest = g;
            while (rest >= 4) {
                for (int base = 0; base < g; base += 4 * stride)
                    for (int o = 0; o < stride; ++o) {
                        double a0 = buf[base + o], a1 = buf[base + o + stride];
                        double a2 = buf[base + o + 2 * stride], a3 = buf[base + o + 3 * stride];
                        double s = a0 + a1 + a2 + a3;
                        buf[base + o] = s - 2.0 * a3;
                        buf[base + o + stride] = s - 2.0 * a2;
                        buf[base + o + 2 * stride] = s - 2.0 * a1;
                        buf[base + o + 3 * stride] = s - 2.0 * a0;
                    }
                stride *= 4;
                rest >>= 2;
            }
            if (rest == 2)
                for (int o = 0; o < stride; ++o) {
                    double a0 = buf[o], a1 = buf[o + stride];
                    buf[o] = a0 + a1;
                    buf[o + stride] = a0 - a1;
                }
            /* g <= 256 and power-of-4 scale is exact; for G=2*4^p the product is rounded in
             * double before the single fp16 rounding (double rounding cannot occur: the double
             * result carries >= 40 more bits than fp16). */
            for (int j = 0; j < g; ++j) tmp_out[c0 + j] = (float)(buf[j] * inv);
        }
        for (int64_t c = 0; c < k; ++c) out[r * k + c] = qlo_f32_to_f16(tmp_out[c]);
    }
    free(tmp_in); free(tmp_out); free(buf);
    return 0;
}

/* ------------------------------------------------------------------------------------------
 * W4A8 / W6A8 (AsymW4A8Int8 storage; weight_error_app.py:145-166, 326-339).
 * ---------------------------------------------------------------------------------------- */

/* Unpack codes: 4-bit plane byte j = code[2j] | code[2j+1] << 4 over K/2 bytes; for 6 bits a
 * second plane follows with byte j = sum_i ((code[4j+i] >> 4) & 3) << 2i over K/4 bytes. */
void qlo_unpack_codes(const uint8_t* q, int64_t n, int64_t k, int bits, int32_t* codes) {
    int64_t cols = k * bits / 8;
    for (int64_t r = 0; r < n; ++r) {
        const uint8_t* row = q + r * cols;
        for (int64_t c = 0; c < k; ++c) {
            int v = (row[c >> 1] >> (4 * (c & 1))) & 0xF;
            if (bits == 6) v |= ((row[k / 2 + (c >> 2)] >> (2 * (c & 3))) & 3) << 4;
            codes[r * k + c] = v;
        }
    }
}

/* Decode to the int8 grid (weight_error_app.py:326-337):
 *   value = codebook[code] (fp32) or float(code - 2^(bits-1));
 *   w8 = clamp(rne(value * float(s_rel[n, c/gs])), -127, 127).
 * s_rel is given as fp32 values (already widened from e4m3 or fp16 storage). */
void qlo_w4a8_int8_grid(const uint8_t* q, const float* s_rel, const float* codebook,
                        int64_t n, int64_t k, int bits, int gs, int8_t* w8) {
    int32_t* codes = (int32_t*)malloc(sizeof(int32_t) * (size_t)k);
    int64_t groups = k / gs;
    for (int64_t r = 0; r < n; ++r) {
        qlo_unpack_codes(q + r * (k * bits / 8), 1, k, bits, codes);
        for (int64_t c = 0; c < k; ++c) {
            float v = codebook ? codebook[codes[c]] : (float)(codes[c] - (1 << (bits - 1)));
            float p = v * s_rel[r * groups + c / gs];
            float t = rne(p);
            if (t < -127.0f) t = -127.0f;
            if (t > 127.0f) t = 127.0f;
            w8[r * k + c] = (int8_t)t;
        }
    }
    free(codes);
}

/* Rotated-basis fp32 weight: float(w8) * s_channel[n] (weight_error_app.py:338). */
void qlo_w4a8_dequantize_rotated(const uint8_t* q, const float* s_rel, const float* s_channel,
                                 const float* codebook, int64_t n, int64_t k, int bits, int gs, float* out) {
    int8_t* w8 = (int8_t*)malloc((size_t)(n * k));
    qlo_w4a8_int8_grid(q, s_rel, codebook, n, k, bits, gs, w8);
    for (int64_t r = 0; r < n; ++r)
        for (int64_t c = 0; c < k; ++c) out[r * k + c] = (float)w8[r * k + c] * s_channel[r];
    free(w8);
}

/* ------------------------------------------------------------------------------------------
 * Dense linear over dequantized operands, y = x @ w^T, accumulated in double.
 * ---------------------------------------------------------------------------------------- */
void qlo_linear_f64(const float* x, const float* w, const float* bias, int64_t m, int64_t n, int64_t k, double* y) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            double acc = 0.0;
            const float* xr = x + i * k;
            const float* wr = w + j * k;
            for (int64_t c = 0; c < k; ++c) acc += (double)xr[c] * (double)wr[c];
            if (bias) acc += (double)bias[j];
            y[i * n + j] = acc;
        }
}

/* Exact int8 x int8 -> int64 accumulation, the check for the int32 MFMA accumulators. */
void qlo_int8_gemm_i64(const int8_t* a, const int8_t* b, int64_t m, int64_t n, int64_t k, int64_t* c) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            int64_t acc = 0;
            for (int64_t t = 0; t < k; ++t) acc += (int64_t)a[i * k + t] * (int64_t)b[j * k + t];
            c[i * n + j] = acc;
        }
}
