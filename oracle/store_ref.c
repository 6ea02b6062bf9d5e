/*
 * oracle/store_ref.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C, IEEE-fp32 restatement of the reference's quantize-on-write store
 * (per-token min/step 4-bit packing into the paged [num_blocks, block_size,
 * KV, D+8] uint8 cache).  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this; the product never does.
 *
 * Follows kernels/kv_dequant_kernels.cuh:816-919 (kv_quantize_store_kernel):
 *   - min/max over the D values of one (token, kv_head) row, NaN-ignoring like
 *     fminf/fmaxf (:838-852, :870-883);
 *   - step = (max - min) / 15.0f, replaced by 1.0f when !(step > 0) (:853-854);
 *   - code = clamp((int)((x - min) / step + 0.5f), 0, 15) with fp32 IEEE ops
 *     and truncation toward zero (:861-864);
 *   - byte j = code[2j] | code[2j+1] << 4 (:865);
 *   - slot base = ((slot / bs) * bs + slot % bs) * KV + kv_head, times D+8;
 *     slot < 0 is skipped (:901-905);
 *   - K bytes at [0, D/2), V bytes at [D/2, D), fp16 (round-to-nearest-even)
 *     k_min, k_step, v_min, v_step at byte offsets D, D+2, D+4, D+6 (:907-918).
 * The float->int conversion follows the GPU convert instruction rather than C's
 * (undefined) cast: NaN -> 0, out-of-range values saturate.
 *
 * Signed zeros: when the smallest value of a row is a zero and the row holds
 * both -0 and +0, the minimum is -0 (and the maximum +0).  This matches the
 * total order -0 < +0 used by the HIP kernel; the reference's tree of fminf
 * calls leaves that case to the order of its reduction.
 *
 * All-NaN rows: the reference reduces over a 128-thread block in which
 * threads d >= D hold +inf (min) / -inf (max) (:838-843).  fminf ignores NaN,
 * so an all-NaN row gives min = NaN when D == 128 (no padding threads) and
 * min = +inf, max = -inf when D < 128.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, x86-64 SSE arithmetic).
 */
#include <stdint.h>
#include <string.h>
#include <math.h>

static float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {                         /* subnormal: man * 2^-24, exact in fp32 */
            float v = (float)man * (1.0f / 16777216.0f);
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* fp32 -> fp16, round to nearest, ties to even; NaN -> canonical quiet NaN. */
uint16_t oracle_float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);           /* NaN */
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);          /* rounds to inf */
    if (ax < 0x38800000u) {                                             /* fp16 subnormal or zero */
        /* value = ax as float; fp16 subnormal unit is 2^-24 */
        float a;
        memcpy(&a, &ax, 4);
        float scaled = a * 16777216.0f;             /* exact: power-of-two scale */
        /* round scaled to nearest integer, ties to even (scaled < 1024) */
        float fl = floorf(scaled);
        float rem = scaled - fl;                    /* exact */
        uint32_t m = (uint32_t)fl;
        if (rem > 0.5f || (rem == 0.5f && (m & 1u))) m += 1u;
        return (uint16_t)(sign | m);                /* m == 1024 gives min normal */
    }
    uint32_t exp = ((ax >> 23) - 112u);
    uint32_t man = ax & 0x7fffffu;
    uint32_t hm = man >> 13;
    uint32_t rest = man & 0x1fffu;
    uint32_t h = (exp << 10) | hm;
    if (rest > 0x1000u || (rest == 0x1000u && (hm & 1u))) h += 1u;    /* carry may bump the exponent */
    return (uint16_t)(sign | h);
}

float oracle_half_to_float(uint16_t h) { return half_to_float(h); }

/* GPU float->int32 conversion: truncate toward zero, NaN -> 0, saturate. */
static int32_t gpu_f2i(float v) {
    if (v != v) return 0;
    if (v >= 2147483648.0f) return 2147483647;
    if (v <= -2147483648.0f) return (int32_t)0x80000000u;
    return (int32_t)v;
}

static float fmin_total(float a, float b) {     /* NaN-ignoring min with -0 < +0 */
    if (a != a) return b;
    if (b != b) return a;
    if (a == b) return signbit(a) ? a : b;
    return a < b ? a : b;
}

static float fmax_total(float a, float b) {     /* NaN-ignoring max with -0 < +0 */
    if (a != a) return b;
    if (b != b) return a;
    if (a == b) return signbit(a) ? b : a;
    return a > b ? a : b;
}

/* Quantize one row of D fp16 values into D/2 packed bytes.
 * Returns the fp32 min and (guarded) step used for the codes. */
void oracle_quantize_row(const uint16_t* row, int D, uint8_t* packed,
                         float* min_out, float* step_out) {
    float mn = NAN, mx = NAN;                       /* NaN is the identity of fmin_total */
    for (int d = 0; d < D; ++d) {
        float v = half_to_float(row[d]);
        mn = fmin_total(mn, v);
        mx = fmax_total(mx, v);
    }
    if (D < 128) {                                  /* the reference's padding threads */
        mn = fmin_total(mn, INFINITY);
        mx = fmax_total(mx, -INFINITY);
    }
    volatile float diff = mx - mn;                  /* keep every op a separate fp32 rounding */
    volatile float step = diff / 15.0f;
    float st = step;
    if (!(st > 0.0f)) st = 1.0f;
    for (int j = 0; j < D / 2; ++j) {
        int32_t c[2];
        for (int t = 0; t < 2; ++t) {
            float x = half_to_float(row[2 * j + t]);
            volatile float num = x - mn;
            volatile float quo = num / st;
            volatile float shifted = quo + 0.5f;
            int32_t q = gpu_f2i(shifted);
            c[t] = q < 0 ? 0 : (q > 15 ? 15 : q);
        }
        packed[j] = (uint8_t)(c[0] | (c[1] << 4));
    }
    *min_out = mn;
    *step_out = st;
}

/* Full store: key/value [N, KV, D] fp16 bits, cache [num_slots, KV, D+8] bytes,
 * slot_mapping [N] int64.  Slots < 0 or >= num_slots are skipped.
 * block_size only matters through slot = block * block_size + pos, which makes
 * the flat slot index equal to the slot id itself. */
void oracle_quantize_store(const uint16_t* key, const uint16_t* value, uint8_t* cache,
                           const int64_t* slot_mapping, int N, int KV, int D,
                           int block_size, int64_t num_slots) {
    const int SLOT = D + 8;
    for (int t = 0; t < N; ++t) {
        int64_t slot = slot_mapping[t];
        if (slot < 0 || slot >= num_slots) continue;
        int64_t blk = slot / block_size, pos = slot % block_size;
        for (int h = 0; h < KV; ++h) {
            uint8_t* dst = cache + ((blk * block_size + pos) * KV + h) * (int64_t)SLOT;
            float kmin, kstep, vmin, vstep;
            oracle_quantize_row(key + ((int64_t)t * KV + h) * D, D, dst, &kmin, &kstep);
            oracle_quantize_row(value + ((int64_t)t * KV + h) * D, D, dst + D / 2, &vmin, &vstep);
            uint16_t r[4] = {oracle_float_to_half(kmin), oracle_float_to_half(kstep),
                             oracle_float_to_half(vmin), oracle_float_to_half(vstep)};
            for (int i = 0; i < 4; ++i) {               /* little-endian fp16 */
                dst[D + 2 * i] = (uint8_t)(r[i] & 0xffu);
                dst[D + 2 * i + 1] = (uint8_t)(r[i] >> 8);
            }
        }
    }
}
