/* C restatement of the dropout RNG -- TEST INFRASTRUCTURE ONLY.
 *
 * Same algorithm as oracle/philox.py (which documents it): Philox4x32-10
 * (Salmon et al., SC'11) with Triton's tl.rand conventions
 * (triton/language/random.py: key = (lo32 seed, hi32 seed), counter =
 * (lo32 c, hi32 c, 0, 0), u = fp32(fold(int32(x0))) * 4.6566127342e-10f),
 * and the dropout counter c = offset + ((b*H + h)*Sq + i)*Sk + j that the
 * reference's forward_kernel.py:110-111,200 intends (row index restored).
 * It exists for speed: full-size (10^8-element) bit-exact mask checks.
 * Built by oracle/Makefile into oracle/_build/liboracle.so; never linked into
 * the product library.
 */
#include <stdint.h>

static inline void philox_round(uint32_t c[4], const uint32_t k[2]) {
    uint64_t pa = (uint64_t)0xD2511F53u * c[0];
    uint64_t pb = (uint64_t)0xCD9E8D57u * c[2];
    uint32_t n0 = (uint32_t)(pb >> 32) ^ c[1] ^ k[0];
    uint32_t n2 = (uint32_t)(pa >> 32) ^ c[3] ^ k[1];
    c[0] = n0; c[1] = (uint32_t)pb; c[2] = n2; c[3] = (uint32_t)pa;
}

void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c[4] = {ctr[0], ctr[1], ctr[2], ctr[3]};
    uint32_t k[2] = {key[0], key[1]};
    for (int r = 0; r < 10; ++r) {
        philox_round(c, k);
        k[0] += 0x9E3779B9u;
        k[1] += 0xBB67AE85u;
    }
    out[0] = c[0]; out[1] = c[1]; out[2] = c[2]; out[3] = c[3];
}

static inline float uniform_from(uint64_t seed, uint64_t ctr64) {
    uint32_t ctr[4] = {(uint32_t)ctr64, (uint32_t)(ctr64 >> 32), 0u, 0u};
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t out[4];
    oracle_philox4x32_10(ctr, key, out);
    int32_t x = (int32_t)out[0];
    if (x < 0) x = -x - 1; /* x >= -2^31, so -x - 1 never overflows */
    return (float)x * 4.6566127342e-10f;
}

void oracle_rand(uint64_t seed, const uint64_t* ctr, int64_t n, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) out[i] = uniform_from(seed, ctr[i]);
}

/* keep[b][h][i][j] = rand(seed, offset + ((b*H+h)*Sq + i)*Sk + j) > p */
void oracle_dropout_keep_mask(uint64_t seed, uint64_t offset, int32_t B, int32_t H,
                              int32_t Sq, int32_t Sk, float p, uint8_t* keep) {
    int64_t rows = (int64_t)B * H * Sq;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t j = 0; j < Sk; ++j) {
            uint64_t c = offset + (uint64_t)(r * (int64_t)Sk + j);
            keep[r * (int64_t)Sk + j] = uniform_from(seed, c) > p ? 1 : 0;
        }
    }
}
