/* C restatement of the integer and byte parts of the MoE step (test infrastructure).
 *
 * This is the checker, never the product: tests and the smoke entry load it
 * through ctypes (oracle/cdecode.py). It is written independently of the
 * torch restatement in moe_ref.py so that the two pin each other.
 *
 *   orc_mxfp4_decode   MXFP4 -> FP32 bit patterns, restating
 *                      megabench/tasks/quantization.py:40-51 by bit
 *                      construction from the OCP MX v1.0 E2M1 / E8M0
 *                      definitions (no value table).
 *   orc_topk_sorted    top-k selection of megabench/tasks/kimi.py:310,316:
 *                      k largest per row (NaN largest, lowest index first on
 *                      ties), returned in ascending expert order.
 *   orc_group          the expert grouping of kimi.py:319-320: per expert in
 *                      ascending order, its (row, slot) pairs in ascending row
 *                      order (a counting sort).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* E2M1 code -> FP32 bit pattern of the unscaled value.
 * sign = bit 3, exponent = bits 2..1 (bias 1), mantissa = bit 0.
 * exponent 0: subnormal, value m * 2^-1; otherwise 2^(e-1) * (1 + m/2). */
static uint32_t e2m1_bits(unsigned code) {
    unsigned s = (code >> 3) & 1u, e = (code >> 1) & 3u, m = code & 1u;
    uint32_t sign = s << 31;
    if (e == 0) {
        if (m == 0) return sign;                 /* +0.0 / -0.0 */
        return sign | (126u << 23);              /* 0.5 = 2^-1 */
    }
    /* 2^(e-1) * (1 + m/2): biased exponent (e - 1) + 127, mantissa MSB = m */
    return sign | ((e - 1u + 127u) << 23) | (m << 22);
}

/* Multiply an FP32 value given by bits by 2^(scale-127), exactly as an IEEE
 * multiply by a power of two rounds (the values here have at most two
 * significant bits, so every finite result is exact). */
static uint32_t scale_bits(uint32_t v, unsigned scale) {
    if (scale == 255u) return 0x7FC00000u;       /* E8M0 NaN -> canonical quiet NaN */
    if ((v & 0x7FFFFFFFu) == 0) return v;        /* signed zero stays */
    int32_t e = (int32_t)((v >> 23) & 0xFFu);    /* inputs are normal: 0.5 .. 6 */
    uint32_t sign = v & 0x80000000u;
    uint32_t mant = v & 0x7FFFFFu;
    int32_t ne = e + (int32_t)scale - 127;
    if (ne >= 255) return sign | 0x7F800000u;    /* overflow -> infinity */
    if (ne >= 1) return sign | ((uint32_t)ne << 23) | mant;
    /* subnormal result: shift the 24-bit significand right by (1 - ne) */
    uint32_t sig = (1u << 23) | mant;
    int shift = 1 - ne;
    if (shift > 24) return sign;                 /* cannot happen for scale >= 0 */
    return sign | (sig >> shift);                /* exact: low bits are zero here */
}

/* blocks: n_blocks x 16 bytes, scales: n_blocks bytes, out: n_blocks x 32 words */
void orc_mxfp4_decode(const uint8_t *blocks, const uint8_t *scales, int64_t n_blocks, uint32_t *out) {
    for (int64_t b = 0; b < n_blocks; ++b) {
        unsigned s = scales[b];
        for (int j = 0; j < 16; ++j) {
            uint8_t byte = blocks[b * 16 + j];
            out[b * 32 + 2 * j] = scale_bits(e2m1_bits(byte & 15u), s);
            out[b * 32 + 2 * j + 1] = scale_bits(e2m1_bits(byte >> 4), s);
        }
    }
}

/* a ranks before b: NaN first, then larger value, then lower index */
static int ranks_before(float va, int ia, float vb, int ib) {
    int na = isnan(va), nb = isnan(vb);
    if (na != nb) return na;
    if (!na && va != vb) return va > vb;
    return ia < ib;
}

/* values: rows x n (row-major); out: rows x k expert ids, ascending */
void orc_topk_sorted(const float *values, int64_t rows, int32_t n, int32_t k, int64_t *out) {
    for (int64_t r = 0; r < rows; ++r) {
        const float *v = values + r * n;
        int64_t *o = out + r * k;
        for (int32_t t = 0; t < k; ++t) {
            int best = -1;
            for (int32_t i = 0; i < n; ++i) {
                int taken = 0;
                for (int32_t u = 0; u < t; ++u) taken |= (o[u] == i);
                if (taken) continue;
                if (best < 0 || ranks_before(v[i], i, v[best], best)) best = i;
            }
            o[t] = best;
        }
        /* insertion sort ascending */
        for (int32_t a = 1; a < k; ++a) {
            int64_t key = o[a];
            int32_t b = a - 1;
            while (b >= 0 && o[b] > key) { o[b + 1] = o[b]; --b; }
            o[b + 1] = key;
        }
    }
}

/* ids: rows x k expert ids (any order, distinct per row, in [0, experts)).
 * counts[experts], offsets[experts + 1]; pair_row / pair_slot[rows * k]:
 * pairs grouped by ascending expert, ascending row inside an expert. */
void orc_group(const int64_t *ids, int64_t rows, int32_t k, int32_t experts,
               int32_t *counts, int32_t *offsets, int32_t *pair_row, int32_t *pair_slot) {
    memset(counts, 0, sizeof(int32_t) * (size_t)experts);
    for (int64_t i = 0; i < rows * k; ++i) counts[ids[i]]++;
    offsets[0] = 0;
    for (int32_t e = 0; e < experts; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int32_t fill[experts > 0 ? experts : 1];
    for (int32_t e = 0; e < experts; ++e) fill[e] = offsets[e];
    for (int64_t r = 0; r < rows; ++r)
        for (int32_t s = 0; s < k; ++s) {
            int64_t e = ids[r * k + s];
            int32_t p = fill[e]++;
            pair_row[p] = (int32_t)r;
            pair_slot[p] = s;
        }
}
