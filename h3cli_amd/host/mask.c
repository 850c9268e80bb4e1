/* Synthetic block-sparse attention mask of the benchmark's joint audio-video
 * sequence (no reference counterpart: the reference routes blocks with a learned
 * SubBlock router, src/cuda/cuda_subblock.cu:256-324, whose output is the same
 * kind of kept-block map).
 *
 * mask[qb * B + kb] (B = ceil(seq / block)) is 1 when any of:
 *   - qb == kb (the diagonal);
 *   - both blocks hold audio rows (rows >= video_rows): all audio<->audio kept;
 *   - u(qb, kb) < density, u = splitmix64((seed << 40) + qb * B + kb) / 2^64.
 */
#include "h3_hip_ext.h"
#include <stdint.h>

static uint64_t splitmix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

unsigned h3_hip_synthetic_block_mask(uint8_t *mask, unsigned seq, unsigned video_rows,
                                     unsigned block, double density, uint64_t seed) {
    if (!mask || !seq || !block || video_rows > seq || !(density >= 0.0 && density <= 1.0)) return 0;
    unsigned blocks = (seq + block - 1) / block, kept = 0;
    /* A block holds audio rows when its last row is >= video_rows. */
    for (unsigned qb = 0; qb < blocks; qb++) {
        unsigned q_last = qb * block + block - 1;
        int q_audio = q_last >= video_rows && video_rows < seq;
        for (unsigned kb = 0; kb < blocks; kb++) {
            unsigned k_last = kb * block + block - 1;
            int k_audio = k_last >= video_rows && video_rows < seq;
            double u = (double)(splitmix64((seed << 40) + (uint64_t)qb * blocks + kb) >> 11) * 0x1.0p-53;
            uint8_t keep = qb == kb || (q_audio && k_audio) || u < density;
            mask[(size_t)qb * blocks + kb] = keep;
            kept += keep;
        }
    }
    return kept;
}
