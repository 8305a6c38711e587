/* C restatement of the reference's weight decoders and an fp64 matvec —
 * TEST INFRASTRUCTURE ONLY (tests/, smoke() and bench.py's cpu_baseline leg).
 *
 * Written independently of the numpy oracle (binary16 is decoded by hand from
 * its bit fields, not through a library conversion) so that the two
 * restatements cross-check each other bit-for-bit:
 *   GF4  w = (4 - (c ^ 4)) * 0.25 * s,  s = binary16(b << 8)   tools/qw35_cook_common.py:54-56,79,115-119
 *   q8_0 w = d * qs[i]                                         qw35-server/src/metal/qw35_types.metal:24-36
 *   Q4_K w = d * sc_j * q - dmin * m_j                         qw35-server/src/metal/qw35_matvec.metal:2-12,
 *                                                              qw35_types.metal:70-83
 *   Q6_K w = d * sc[e/16] * (q - 32), q = ql nibble | qh bits << 4
 *                                                              qw35_matvec.metal:458-542 (bit extraction),
 *                                                              qw35_types.metal:17-22 (block)
 *   Q5_K w = d * sc_j * q - dmin * m_j, q = nibble | bit j of qh[e % 32] << 4
 *                                                              qw35_matvec.metal:40-62, qw35_types.metal:9-15
 *   GF2  w = (q * fl(2/3) - 1) * s, 2-bit q, 80-byte super-blocks of 16 words + 16 scale bytes
 *                                                              qw35_gf2.metal:1-50
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

static float half_bits_to_float(uint16_t h) {
    const int sign = (h >> 15) & 1;
    const int e = (h >> 10) & 0x1F;
    const int m = h & 0x3FF;
    float v;
    if (e == 0) {
        v = ldexpf((float)m, -24); /* subnormal: m * 2^-24 */
    } else if (e == 31) {
        v = m ? NAN : INFINITY;
    } else {
        v = ldexpf((float)(1024 + m), e - 25); /* (1 + m/1024) * 2^(e-15) */
    }
    return sign ? -v : v;
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

void qw35o_gf4_dequant(const uint32_t *words, size_t n_words, float *out) {
    for (size_t g = 0; g < n_words; ++g) {
        const uint32_t w = words[g];
        const float s = half_bits_to_float((uint16_t)((w & 0xFFu) << 8));
        for (int i = 0; i < 8; ++i) {
            const uint32_t c = (w >> (8 + 3 * i)) & 7u;
            const uint32_t q = c ^ 4u;
            out[8 * g + i] = (4.0f - (float)q) * 0.25f * s;
        }
    }
}

void qw35o_q8_0_dequant(const uint8_t *raw, size_t n_blocks, float *out) {
    for (size_t b = 0; b < n_blocks; ++b) {
        const uint8_t *blk = raw + 34 * b;
        const float d = half_bits_to_float(rd16(blk));
        for (int i = 0; i < 32; ++i) out[32 * b + i] = d * (float)(int8_t)blk[2 + i];
    }
}

static void scale_min_k4(int j, const uint8_t *q, int *sc, int *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

void qw35o_q4_k_dequant(const uint8_t *raw, size_t n_blocks, float *out) {
    for (size_t b = 0; b < n_blocks; ++b) {
        const uint8_t *blk = raw + 144 * b;
        const float d = half_bits_to_float(rd16(blk));
        const float dmin = half_bits_to_float(rd16(blk + 2));
        const uint8_t *scales = blk + 4;
        const uint8_t *qs = blk + 16;
        for (int e = 0; e < 256; ++e) {
            const int j = e / 32;
            int sc, m;
            scale_min_k4(j, scales, &sc, &m);
            const uint8_t byte = qs[(j / 2) * 32 + (e % 32)];
            const int q = (j & 1) ? (byte >> 4) : (byte & 0x0F);
            const float dsc = d * (float)sc;
            const float mm = dmin * (float)m;
            out[256 * b + e] = dsc * (float)q - mm;
        }
    }
}

/* Q6_K, written from the reference GEMV's extraction: for each half ip and
 * position l in 0..31, bytes ql[64ip + l], ql[64ip + 32 + l], qh[32ip + l]
 * give elements 128ip + l + {0, 32, 64, 96}. */
void qw35o_q6_k_dequant(const uint8_t *raw, size_t n_blocks, float *out) {
    for (size_t b = 0; b < n_blocks; ++b) {
        const uint8_t *blk = raw + 210 * b;
        const uint8_t *ql = blk;
        const uint8_t *qh = blk + 128;
        const int8_t *sc = (const int8_t *)(blk + 192);
        const float d = half_bits_to_float(rd16(blk + 208));
        for (int ip = 0; ip < 2; ++ip) {
            for (int l = 0; l < 32; ++l) {
                const int a = ql[64 * ip + l], c = ql[64 * ip + 32 + l], h = qh[32 * ip + l];
                const int q[4] = {(a & 15) | ((h & 3) << 4), (c & 15) | (((h >> 2) & 3) << 4),
                                  (a >> 4) | (((h >> 4) & 3) << 4), (c >> 4) | (((h >> 6) & 3) << 4)};
                for (int j = 0; j < 4; ++j) {
                    const int e = 128 * ip + 32 * j + l;
                    out[256 * b + e] = (d * (float)sc[e / 16]) * (float)(q[j] - 32);
                }
            }
        }
    }
}

/* Q5_K: the Q4_K block with 32 bytes of fifth code bits between the scales
 * and the nibbles (d, dmin, scales[12], qh[32], qs[128] = 176 bytes). */
void qw35o_q5_k_dequant(const uint8_t *raw, size_t n_blocks, float *out) {
    for (size_t b = 0; b < n_blocks; ++b) {
        const uint8_t *blk = raw + 176 * b;
        const float d = half_bits_to_float(rd16(blk));
        const float dmin = half_bits_to_float(rd16(blk + 2));
        const uint8_t *scales = blk + 4;
        const uint8_t *qh = blk + 16;
        const uint8_t *qs = blk + 48;
        for (int e = 0; e < 256; ++e) {
            const int j = e / 32;
            int sc, m;
            scale_min_k4(j, scales, &sc, &m);
            const uint8_t byte = qs[(j / 2) * 32 + (e % 32)];
            const int q = ((j & 1) ? (byte >> 4) : (byte & 0x0F)) | (((qh[e % 32] >> j) & 1) << 4);
            const float dsc = d * (float)sc;
            const float mm = dmin * (float)m;
            out[256 * b + e] = dsc * (float)q - mm;
        }
    }
}

/* GF2: per 256 columns, 16 little-endian code words (code i of word w is
 * column 16w + i, bits 2i..2i+1) then their 16 e5m2 scale bytes. */
void qw35o_gf2_dequant(const uint8_t *raw, size_t n_blocks, float *out) {
    const float two_thirds = 2.0f / 3.0f;
    for (size_t b = 0; b < n_blocks; ++b) {
        const uint8_t *blk = raw + 80 * b;
        for (int w = 0; w < 16; ++w) {
            const uint32_t word = (uint32_t)blk[4 * w] | ((uint32_t)blk[4 * w + 1] << 8) |
                                  ((uint32_t)blk[4 * w + 2] << 16) | ((uint32_t)blk[4 * w + 3] << 24);
            const float s = half_bits_to_float((uint16_t)(blk[64 + w] << 8));
            for (int i = 0; i < 16; ++i) {
                const float q = (float)((word >> (2 * i)) & 3u);
                const float level = q * two_thirds - 1.0f;
                out[256 * b + 16 * w + i] = level * s;
            }
        }
    }
}

/* y[b][r] = sum_k w[r][k] * x[b][k] in double. */
void qw35o_matvec_f64(const float *w, size_t rows, size_t k, const float *x, size_t nb, double *y) {
    for (size_t b = 0; b < nb; ++b) {
        for (size_t r = 0; r < rows; ++r) {
            double acc = 0.0;
            const float *wr = w + r * k;
            const float *xb = x + b * k;
            for (size_t i = 0; i < k; ++i) acc += (double)wr[i] * (double)xb[i];
            y[b * rows + r] = acc;
        }
    }
}
