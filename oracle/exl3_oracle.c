/* C restatement of the EXL3 trellis decode -- TEST INFRASTRUCTURE ONLY (the checker, never the product).
 *
 * Restates core/src/trellis_core/reference.py:
 *   codebook_lut        52-73   (integer hash + fp16 arithmetic with a hand-written round-to-nearest-even)
 *   _state_index /      80-99   (here as a 64-bit funnel over two stream words instead of the reference's
 *   decode_states                bit gather, so the two restatements share no code path)
 *   tensor_core_perm    30-45   (as the closed form of xpu/csrc/exl3_esimd.h:6-8)
 *   reconstruct_inner   102-115
 * Built by oracle/Makefile into oracle/_build/libexl3_oracle.so and loaded by the tests with ctypes.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* ---- fp16 <-> double, written from the IEEE-754 binary16 definition ---- */
static double f16_to_f64(uint16_t h) {
    int sign = h >> 15, exp = (h >> 10) & 0x1F, man = h & 0x3FF;
    double v;
    if (exp == 0) v = ldexp((double)man, -24);
    else if (exp == 31) v = man ? NAN : INFINITY;
    else v = ldexp((double)(man | 0x400), exp - 25);
    return sign ? -v : v;
}

/* round a double to the nearest binary16, ties to even */
static uint16_t f64_to_f16_rne(double v) {
    uint16_t sign = 0;
    if (isnan(v)) return 0x7E00;
    if (signbit(v)) { sign = 0x8000; v = -v; }
    if (v == 0.0) return sign;
    int e;
    frexp(v, &e);            /* v = f * 2^e, f in [0.5, 1) */
    int exp16 = e - 1 + 15;  /* biased exponent of the leading bit */
    double q;                /* value in units of the target ulp */
    if (exp16 <= 0) {        /* subnormal range: ulp = 2^-24 */
        q = ldexp(v, 24);
    } else {
        q = ldexp(v, 10 - (e - 1));   /* mantissa with 10 fraction bits */
    }
    double r = nearbyint(q);  /* default rounding mode: to nearest, ties to even */
    uint32_t bits;
    if (exp16 <= 0) {
        bits = (uint32_t)r;   /* may round up into the smallest normal: encoding stays correct */
    } else {
        uint32_t m = (uint32_t)r;     /* in [1024, 2048] */
        if (m == 2048) { m = 1024; exp16++; }
        if (exp16 >= 31) return sign | 0x7C00;
        bits = ((uint32_t)exp16 << 10) | (m - 1024);
    }
    return sign | (uint16_t)bits;
}

uint16_t exl3_oracle_f64_to_f16(double v) { return f64_to_f16_rne(v); }
double exl3_oracle_f16_to_f64(uint16_t h) { return f16_to_f64(h); }

/* ---- codebooks: 16-bit state -> fp16 bits ---- */
uint16_t exl3_oracle_codebook(int cb, uint32_t state) {
    uint32_t s = state & 0xFFFFu;
    if (cb == 2) {  /* mul1: byte sum of the product, as fp16 1024 + bsum, one fused multiply-add */
        uint32_t x = s * 0x83DCD12Du;
        uint32_t bsum = (x & 0xFF) + ((x >> 8) & 0xFF) + ((x >> 16) & 0xFF) + (x >> 24);
        double h = f16_to_f64((uint16_t)(0x6400u + bsum));
        return f64_to_f16_rne(h * f16_to_f64(0x1EEE) + f16_to_f64(0xC931));
    }
    uint32_t x = cb == 0 ? s * 89226354u + 64248484u : s * 0xCBAC1FEDu;
    x = (x & 0x8FFF8FFFu) ^ 0x3B603B60u;
    return f64_to_f16_rne(f16_to_f64((uint16_t)(x & 0xFFFF)) + f16_to_f64((uint16_t)(x >> 16)));
}

void exl3_oracle_codebook_lut(int cb, uint16_t* out) {
    for (uint32_t s = 0; s < 65536u; s++) out[s] = exl3_oracle_codebook(cb, s);
}

/* ---- one tile: 16K int16 -> 256 states in stream order ---- */
void exl3_oracle_decode_tile(const int16_t* tile, int K, uint32_t* states) {
    const int nwords = 8 * K, nbits = 256 * K;
    uint32_t w[64];
    for (int m = 0; m < nwords; m++)
        w[m] = (uint32_t)(uint16_t)tile[2 * m] | ((uint32_t)(uint16_t)tile[2 * m + 1] << 16);
    for (int t = 0; t < 256; t++) {
        /* the window is the 16 bits ending at bit (t+1)K, circular; bit 0 = MSB of word 0 */
        int end = ((t + 1) * K) % nbits;            /* exclusive end, in [0, nbits) */
        int start = (end - 16 + nbits) % nbits;
        int wi = start / 32, off = start % 32;
        uint64_t hilo = ((uint64_t)w[wi] << 32) | w[(wi + 1) % nwords];
        states[t] = (uint32_t)((hilo >> (48 - off)) & 0xFFFFu);
    }
}

/* tile stream position t -> (row, col), the closed form of xpu/csrc/exl3_esimd.h:6-8 */
static inline int perm_row(int t) { return 8 * ((t >> 1) & 1) + 2 * ((t >> 3) & 3) + (t & 1); }
static inline int perm_col(int t) { return (t >> 5) + 8 * ((t >> 2) & 1); }

void exl3_oracle_perm(int32_t* rows, int32_t* cols) {
    for (int t = 0; t < 256; t++) { rows[t] = perm_row(t); cols[t] = perm_col(t); }
}

/* trellis int16 [tk, tn, 16K] -> W_inner fp16 bits [16 tk, 16 tn] */
void exl3_oracle_reconstruct(const int16_t* trellis, int64_t tk, int64_t tn, int K, int cb, uint16_t* out) {
    static uint16_t lut[3][65536];
    static int lut_ready[3] = {0, 0, 0};
    if (!lut_ready[cb]) { exl3_oracle_codebook_lut(cb, lut[cb]); lut_ready[cb] = 1; }
    const int64_t n = 16 * tn;
    uint32_t st[256];
    for (int64_t i = 0; i < tk; i++)
        for (int64_t j = 0; j < tn; j++) {
            exl3_oracle_decode_tile(trellis + (i * tn + j) * 16 * K, K, st);
            for (int t = 0; t < 256; t++)
                out[(16 * i + perm_row(t)) * n + 16 * j + perm_col(t)] = lut[cb][st[t]];
        }
}
