/*
 * CPU oracle for the NF4 byte/integer arithmetic of the MoE expert path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (moeinfra_amd/) may link,
 * import or call this file; only tests/, the smoke check and the CPU-baseline
 * leg of bench.py use it, and only as the checker.
 *
 * What it restates (reference = ParshwaPatel-07/MoEInfra):
 *   - the NF4 dequantisation executed inside bitsandbytes 0.50.2
 *     `dequantize_4bit` for the state built at transfer/nf4_reconstruct.py:17-54
 *     (blocksize 64 `_NF4_BLOCKSIZE` :9, fp32 absmax, output dtype bf16 `_NF4_DTYPE` :12):
 *         W[i] = bf16_rne( code[q_i] * absmax[i / blocksize] )      (one fp32 multiply)
 *     with q_{2j} in the HIGH nibble of packed byte j and q_{2j+1} in the low nibble;
 *   - the NF4 blockwise quantiser that bitsandbytes runs when an expert built by
 *     model/expert.py:32-63 (compress_statistics=False, quant_type="nf4") is moved to the
 *     GPU (model/loader.py:404-415):  absmax = max|w| per block, x = w * (1/absmax), and
 *     q = the nearest code value, decided by comparing x against the midpoints of
 *     consecutive code values with a strict ">" (x exactly on a midpoint takes the lower code).
 *
 * bitsandbytes is a third-party dependency (pinned bitsandbytes==0.50.2 at
 * requirements.txt:3) that is not vendored and not installed, so its published
 * algorithm is restated here.  Pinned by the tests: the dequant formula (closed forms,
 * an independent torch float32-multiply + bf16 conversion), the codebook (rebuilt from
 * its normal-quantile construction), quantise/dequantise idempotence and the
 * nearest-code property.  Parity unpinned (needs a bitsandbytes-written store): the
 * nibble order, the exact midpoint constants and tie rule of bnb's quantiser.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* float -> bf16, round to nearest even; NaN -> canonical quiet NaN 0x7FC0
 * (the rounding torch's bfloat16 conversion performs). */
uint16_t oracle_bf16_rne(float f)
{
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu) != 0u)
        return (uint16_t)0x7fc0u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float oracle_bf16_to_f32(uint16_t h)
{
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* Dequantise `numel` NF4 values (numel even) into bf16 bit patterns. */
int oracle_nf4_dequant(const uint8_t *packed, const float *absmax, const float *code,
                       int64_t numel, int32_t blocksize, uint16_t *out)
{
    if (numel < 0 || (numel & 1) || blocksize <= 0)
        return -1;
    for (int64_t i = 0; i < numel; i += 2) {
        const uint8_t b = packed[i >> 1];
        out[i] = oracle_bf16_rne(code[b >> 4] * absmax[i / blocksize]);
        out[i + 1] = oracle_bf16_rne(code[b & 15] * absmax[(i + 1) / blocksize]);
    }
    return 0;
}

/* Quantise bf16 bit patterns to packed NF4 + fp32 absmax (ceil(numel/blocksize) blocks). */
int oracle_nf4_quantize(const uint16_t *w, int64_t numel, int32_t blocksize, const float *code,
                        uint8_t *packed, float *absmax)
{
    if (numel < 0 || (numel & 1) || blocksize <= 0 || (blocksize & 1))
        return -1;
    float mid[15];
    for (int i = 0; i < 15; ++i)
        mid[i] = (code[i] + code[i + 1]) * 0.5f;
    const int64_t nblocks = (numel + blocksize - 1) / blocksize;
    for (int64_t b = 0; b < nblocks; ++b) {
        const int64_t lo = b * blocksize;
        const int64_t hi = lo + blocksize < numel ? lo + blocksize : numel;
        float amax = 0.0f;
        for (int64_t i = lo; i < hi; ++i) {
            const float a = fabsf(oracle_bf16_to_f32(w[i]));
            if (a > amax)
                amax = a;
        }
        absmax[b] = amax;
        const float r = amax > 0.0f ? 1.0f / amax : 0.0f;
        for (int64_t i = lo; i < hi; i += 2) {
            uint8_t q[2];
            for (int j = 0; j < 2; ++j) {
                const float x = oracle_bf16_to_f32(w[i + j]) * r;
                int c = 0;
                for (int m = 0; m < 15; ++m)
                    c += x > mid[m];
                q[j] = (uint8_t)c;
            }
            packed[i >> 1] = (uint8_t)((q[0] << 4) | q[1]);
        }
    }
    return 0;
}
