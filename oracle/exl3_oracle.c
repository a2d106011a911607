/*
 * CPU oracle for the EXL3 quantized-matmul path.  TEST INFRASTRUCTURE ONLY:
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library; the product (sglang-exl3_amd/) never does.
 *
 * A plain-C restatement of the reference's host decode and dequant, written
 * from the reference's behaviour (not copied):
 *
 *   - 16-bit window of the tail-biting trellis bitstream
 *       /root/reference/csrc/exl3_dequant.cuh:110-128 (read_window)
 *       /root/reference/csrc/exl3_dequant.cuh:130-135 (decode_weight index)
 *   - codebooks cb0 "3INST", cb1 MCG, cb2 mul1
 *       host, truncating fp16:  csrc/exl3_dequant.cuh:41-55, 57-69, 74-93
 *       device, round-to-nearest: csrc/quant/codebook.cuh:41,53,56-90
 *   - 16x16 tile swizzle: csrc/bindings.cpp:37-76
 *   - 128-point radix-2 Walsh-Hadamard: csrc/exl3_dequant.cuh:137-148
 *   - full dequant (two FWHT passes, scale order, fp16 RNE store):
 *       csrc/bindings.cpp:15-100
 *   - reference CPU matmul (dequant, then fp32 GEMM): csrc/bindings.cpp:144-146
 *   - MoE expert MLP and combine: src/sglang_exl3/exl3.py:562-575 (SwiGLU with
 *     clip, fp32 index_add of w * down)
 *
 * Build: oracle/Makefile (gcc, -ffp-contract=off so every fp32 operation is
 * rounded exactly where the reference rounds it).
 */
#include <stdint.h>
#include <stddef.h>
#include <string.h>
#include <math.h>
#include <stdlib.h>

#define ORC_MCG_MUL 0xCBAC1FEDu
#define ORC_MUL1_MUL 0x83DCD12Du
#define ORC_3INST_MUL 89226354u
#define ORC_3INST_ADD 64248484u
#define ORC_HAD_NORM 0.08838834764831845f

/* ---------------------------------------------------------------- fp16 bits */

float orc_half_to_float(uint16_t h)
{
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
    float f;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in fp32 */
        f = (float)m * 5.9604644775390625e-08f;
        return sign ? -f : f;
    }
    if (e == 31) bits = sign | 0x7f800000u | (m << 13);
    else bits = sign | ((e - 15 + 127) << 23) | (m << 13);
    memcpy(&f, &bits, 4);
    return f;
}

/* Truncating fp32 -> fp16 exactly as the reference host code does it
 * (csrc/exl3_dequant.cuh:41-55), including its handling of values below the
 * normal range (the shift it uses there is kept as written; decoded codebook
 * values never reach that branch, |v| >= 2^-13). */
uint16_t orc_float_to_half_rtz(float v)
{
    uint32_t raw;
    memcpy(&raw, &v, 4);
    uint32_t sign = (raw >> 16) & 0x8000u;
    int e = (int)((raw >> 23) & 0xffu) - 127;
    uint32_t mant = raw & 0x7fffffu;
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    if (e < -14) {
        if (e < -24) return (uint16_t)sign;
        uint32_t m = (mant | 0x800000u) >> (-e - 1);
        return (uint16_t)(sign | (m >> 13));
    }
    return (uint16_t)(sign | ((uint32_t)(e + 15) << 10) | (mant >> 13));
}

/* IEEE round-to-nearest-even fp32 -> fp16 (c10::Half, __float2half_rn). */
uint16_t orc_float_to_half_rne(float v)
{
    uint32_t x;
    memcpy(&x, &v, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds past 65504 */
    if (ax < 0x38800000u) {
        /* result subnormal or zero: units of 2^-24 */
        if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25: rounds to 0 */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e; /* value = m * 2^(e-150); units = m >> (126-e) */
        uint32_t q = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 127 + 15;
    uint32_t m = ax & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

/* ------------------------------------------------------------- bitstream */

/* 16-bit window starting at stream bit `bit` of a tile of `words16` int16
 * entries; the tile is read as little-endian uint32 words, bits are taken
 * MSB-first, and the stream wraps (tail-biting). */
uint16_t orc_read_window(const uint16_t* tile, size_t words16, size_t bit)
{
    size_t nbits = words16 * 16, n32 = words16 / 2;
    bit %= nbits;
    size_t end = bit + 16;
    size_t i0 = (bit / 32) % n32;
    size_t i1 = ((end - 1) / 32) % n32;
    unsigned shift = (unsigned)((((end - 1) / 32) + 1) * 32 - end);
    uint32_t a = (uint32_t)tile[2 * i0] | ((uint32_t)tile[2 * i0 + 1] << 16);
    uint32_t b = (uint32_t)tile[2 * i1] | ((uint32_t)tile[2 * i1 + 1] << 16);
    uint64_t merged = ((uint64_t)a << 32) | b;
    return (uint16_t)((merged >> shift) & 0xffffu);
}

/* Stream bit where the window of value t (0..255) of a K-bit tile starts. */
size_t orc_window_start(int t, int K)
{
    return (size_t)(t + 257) * (size_t)K - 16u;
}

/* -------------------------------------------------------------- codebooks */

static uint32_t masked(uint32_t x) { return (x & 0x8fff8fffu) ^ 0x3b603b60u; }

/* Exact fp32 value of the codebook entry for `state` (every intermediate is
 * exact in fp32: two fp16 halves in [2^-3, 2) for cb0/cb1, an integer
 * multiple of 2^-18 below 2^22 for cb2). */
float orc_codebook_exact(uint16_t state, int cb)
{
    uint32_t x = state;
    if (cb == 0 || cb == 1) {
        x = (cb == 0) ? x * ORC_3INST_MUL + ORC_3INST_ADD : x * ORC_MCG_MUL;
        x = masked(x);
        return orc_half_to_float((uint16_t)x) + orc_half_to_float((uint16_t)(x >> 16));
    }
    x *= ORC_MUL1_MUL;
    uint32_t h = 0x6400u + (x & 0xffu) + ((x >> 8) & 0xffu) + ((x >> 16) & 0xffu) + (x >> 24);
    return orc_half_to_float((uint16_t)h) * orc_half_to_float(0x1eeeu) + orc_half_to_float(0xc931u);
}

/* fp16 bits of the codebook entry: rtz != 0 -> host reference rounding
 * (truncation), rtz == 0 -> CUDA kernel rounding (__hadd/__hfma, RNE). */
uint16_t orc_decode_state(uint16_t state, int cb, int rtz)
{
    float v = orc_codebook_exact(state, cb);
    return rtz ? orc_float_to_half_rtz(v) : orc_float_to_half_rne(v);
}

void orc_codebook_table(int cb, int rtz, uint16_t* out65536)
{
    for (uint32_t s = 0; s < 65536u; ++s) out65536[s] = orc_decode_state((uint16_t)s, cb, rtz);
}

/* ------------------------------------------------------------ tile layout */

/* Position of value t (0..255) inside the 16x16 tile: row = input feature k,
 * column = output feature n (csrc/bindings.cpp:51-75 restated in closed form). */
void orc_tile_pos(int t, int* k, int* n)
{
    int l = t >> 3, j = t & 7;
    *k = 2 * (l & 3) + (j & 1) + 8 * ((j >> 1) & 1);
    *n = (l >> 2) + 8 * (j >> 2);
}

/* Decode one 16*K-word tile into a row-major 16x16 fp16 block. */
void orc_decode_tile(const uint16_t* tile, int K, int cb, int rtz, uint16_t* out256)
{
    for (int t = 0; t < 256; ++t) {
        uint16_t s = orc_read_window(tile, (size_t)16 * K, orc_window_start(t, K));
        int k, n;
        orc_tile_pos(t, &k, &n);
        out256[k * 16 + n] = orc_decode_state(s, cb, rtz);
    }
}

/* --------------------------------------------------------------- hadamard */

void orc_fwht(float* v, int n)
{
    for (int s = 1; s < n; s <<= 1)
        for (int b = 0; b < n; b += 2 * s)
            for (int i = 0; i < s; ++i) {
                float a = v[b + i], c = v[b + s + i];
                v[b + i] = a + c;
                v[b + s + i] = a - c;
            }
}

/* --------------------------------------------------------------- dequant */

/* W[k,n] fp16 bits, bit-exact with the reference host dequant
 * (csrc/bindings.cpp:15-100): decode with truncating fp16 rounding (rtz=1)
 * or, for comparison, with kernel rounding (rtz=0).  trellis is
 * [k/16][n/16][16K] int16.  Returns 0 on success, -1 on a shape error,
 * -2 on allocation failure. */
int orc_dequant(const uint16_t* trellis, const uint16_t* suh, const uint16_t* svh,
                int k, int n, int K, int cb, int rtz, uint16_t* W)
{
    if (k <= 0 || n <= 0 || (k % 128) || (n % 128) || K < 1 || K > 8) return -1;
    size_t words = (size_t)16 * K;
    float* M = (float*)malloc((size_t)k * n * sizeof(float));
    if (!M) return -2;
    uint16_t blk[256];
    for (int kt = 0; kt < k / 16; ++kt)
        for (int nt = 0; nt < n / 16; ++nt) {
            orc_decode_tile(trellis + ((size_t)kt * (n / 16) + nt) * words, K, cb, rtz, blk);
            for (int r = 0; r < 16; ++r)
                for (int c = 0; c < 16; ++c)
                    M[(size_t)(kt * 16 + r) * n + nt * 16 + c] = orc_half_to_float(blk[r * 16 + c]);
        }
    float line[128];
    for (int r0 = 0; r0 < k; r0 += 128)
        for (int c0 = 0; c0 < n; c0 += 128) {
            for (int r = 0; r < 128; ++r) {
                float* row = M + (size_t)(r0 + r) * n + c0;
                memcpy(line, row, sizeof(line));
                orc_fwht(line, 128);
                for (int c = 0; c < 128; ++c) row[c] = line[c] * ORC_HAD_NORM;
            }
            for (int c = 0; c < 128; ++c) {
                for (int r = 0; r < 128; ++r) line[r] = M[(size_t)(r0 + r) * n + c0 + c];
                orc_fwht(line, 128);
                for (int r = 0; r < 128; ++r) {
                    float v = line[r] * ORC_HAD_NORM;
                    v = v * orc_half_to_float(suh[r0 + r]);
                    v = v * orc_half_to_float(svh[c0 + c]);
                    W[(size_t)(r0 + r) * n + c0 + c] = orc_float_to_half_rne(v);
                }
            }
        }
    free(M);
    return 0;
}

/* ---------------------------------------------------------------- matmul */

/* y[m,n] = x[m,k] . W[k,n] with fp16 inputs, fp32 products and fp64
 * accumulation (a tighter reference than the reference's fp32 at::mm).
 * A product of two fp16 values is exact in fp32.  Zero inputs are not
 * skipped, so 0 * inf and 0 * NaN in W give NaN as IEEE arithmetic does. */
void orc_matmul_f16(const uint16_t* x, const uint16_t* W, int m, int k, int n, float* y)
{
    double* acc = (double*)calloc((size_t)n, sizeof(double));
    float* wrow = (float*)malloc((size_t)n * sizeof(float));
    for (int i = 0; i < m; ++i) {
        memset(acc, 0, (size_t)n * sizeof(double));
        for (int kk = 0; kk < k; ++kk) {
            float xv = orc_half_to_float(x[(size_t)i * k + kk]);
            const uint16_t* wr = W + (size_t)kk * n;
            for (int j = 0; j < n; ++j) wrow[j] = orc_half_to_float(wr[j]);
            for (int j = 0; j < n; ++j) acc[j] += (double)(xv * wrow[j]);
        }
        for (int j = 0; j < n; ++j) y[(size_t)i * n + j] = (float)acc[j];
    }
    free(acc);
    free(wrow);
}

/* The reference's CPU exl3_gemv path (csrc/bindings.cpp:144-146):
 * dequant (truncating decode) then an fp32 GEMM.  Used as the timed CPU
 * baseline; accumulation here is fp32 in k order. */
int orc_cpu_gemv(const uint16_t* x, const uint16_t* trellis, const uint16_t* suh,
                 const uint16_t* svh, int m, int k, int n, int K, int cb,
                 uint16_t* W_scratch, float* y)
{
    int rc = orc_dequant(trellis, suh, svh, k, n, K, cb, 1, W_scratch);
    if (rc) return rc;
    float* wrow = (float*)malloc((size_t)n * sizeof(float));
    if (!wrow) return -2;
    for (int i = 0; i < m; ++i) {
        float* yr = y + (size_t)i * n;
        for (int j = 0; j < n; ++j) yr[j] = 0.0f;
        for (int kk = 0; kk < k; ++kk) {
            float xv = orc_half_to_float(x[(size_t)i * k + kk]);
            const uint16_t* wr = W_scratch + (size_t)kk * n;
            for (int j = 0; j < n; ++j) wrow[j] = orc_half_to_float(wr[j]);
            for (int j = 0; j < n; ++j) yr[j] += xv * wrow[j];
        }
    }
    free(wrow);
    return 0;
}

/* Decode-only timing helper: dequant without the matmul. */
int orc_dequant_only(const uint16_t* trellis, const uint16_t* suh, const uint16_t* svh,
                     int k, int n, int K, int cb, uint16_t* W)
{
    return orc_dequant(trellis, suh, svh, k, n, K, cb, 1, W);
}

/* ------------------------------------------------------------- hadamard op */

/* y = fp32 H128 transform of each 128-block of every row, with optional
 * pre-scale (x*pre) and post-scale (*post) vectors of length `cols`, and a
 * global factor r; the semantic of the reference's had_r_128 helper
 * (csrc/quant/hadamard_inner.cuh:150-210). */
void orc_had_rows(const float* x, int rows, int cols, const uint16_t* pre, const uint16_t* post,
                  float r, float* y)
{
    float line[128];
    for (int i = 0; i < rows; ++i)
        for (int c0 = 0; c0 < cols; c0 += 128) {
            for (int c = 0; c < 128; ++c) {
                float v = x[(size_t)i * cols + c0 + c];
                if (pre) v *= orc_half_to_float(pre[c0 + c]);
                line[c] = v;
            }
            orc_fwht(line, 128);
            for (int c = 0; c < 128; ++c) {
                float v = line[c] * r;
                if (post) v *= orc_half_to_float(post[c0 + c]);
                y[(size_t)i * cols + c0 + c] = v;
            }
        }
}

/* --------------------------------------------------------------------- MoE */

/* silu(min(g, L)) * clamp(u, -L, L) in fp32; L <= 0 or non-finite disables
 * the clip (src/sglang_exl3/exl3.py:572; csrc/p2b_moe.cu:283-290). */
float orc_swiglu(float g, float u, float L)
{
    if (L > 0.0f && isfinite(L)) {
        if (g > L) g = L;
        if (u > L) u = L;
        if (u < -L) u = -L;
    }
    return g / (1.0f + expf(-g)) * u;
}
