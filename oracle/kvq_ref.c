/* SPDX-License-Identifier: Apache-2.0
 *
 * Scalar C restatement of the quantized-KV arithmetic -- TEST INFRASTRUCTURE.
 *
 * A second, independent oracle: one element at a time, plain loops, built with
 * -ffp-contract=off so every fp32 operation rounds exactly once, as IEEE and
 * the reference's torch ops do.  Tests use it to pin the vectorized torch
 * oracle (oracle/kvq_oracle.py) bit for bit; the product never links it.
 * Paths are relative to /root/reference, pkg/ = src/vllm_ascend_quantized_kv_cache/.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* pkg/methods/kivi_int4/semantics.py:86-93 -- scale floor applies to the scale. */
static float group_scale(float mn, float mx) {
    float s = (mx - mn) / 15.0f;
    return s < 1.0e-6f ? 1.0e-6f : s;
}

/* semantics.py:95-111 -- floor(x + 0.5): ties round up, not to even. */
static int32_t quantize(float x, float mn, float scale) {
    float t = (x - mn) / scale;
    t = t + 0.5f;
    t = floorf(t);
    if (t < 0.0f) t = 0.0f;
    if (t > 15.0f) t = 15.0f;
    return (int32_t)t;
}

/* Key pack: pkg/ops/triton/kivi_pack.py:161-226.
 * key [T, KVH, D] fp32; slots [T]; caches [NB,KVH,D,Bs/8] / [NB,KVH,D,Bs/G]. */
void ref_pack_key(const float *key, int64_t T, int kvh, int d, const int64_t *slots,
                  int g, int bs, int32_t *kq, float *ks, float *km) {
    for (int64_t t0 = 0; t0 + g <= T; t0 += g) {
        int64_t first = slots[t0];
        if (first < 0) continue;
        int64_t blk = first / bs, off = first % bs;
        for (int h = 0; h < kvh; ++h) {
            for (int c = 0; c < d; ++c) {
                float mn = INFINITY, mx = -INFINITY;
                for (int i = 0; i < g; ++i) {
                    float x = key[((t0 + i) * kvh + h) * d + c];
                    if (x < mn) mn = x;
                    if (x > mx) mx = x;
                }
                float sc = group_scale(mn, mx);
                int64_t srow = ((blk * kvh + h) * d + c);
                ks[srow * (bs / g) + off / g] = sc;
                km[srow * (bs / g) + off / g] = mn;
                for (int w = 0; w < g / 8; ++w) {
                    uint32_t word = 0;
                    for (int lane = 0; lane < 8; ++lane) {
                        float x = key[((t0 + 8 * w + lane) * kvh + h) * d + c];
                        word |= (uint32_t)quantize(x, mn, sc) << (4 * lane);
                    }
                    kq[srow * (bs / 8) + off / 8 + w] = (int32_t)word;
                }
            }
        }
    }
}

/* Value pack: pkg/ops/triton/kivi_pack.py:84-131.
 * value [T, KVH, D] fp32; caches [NB,Bs,KVH,D/8] / [NB,Bs,KVH,D/G]. */
void ref_pack_value(const float *value, int64_t T, int kvh, int d, const int64_t *slots,
                    int g, int bs, int32_t *vq, float *vs, float *vm) {
    for (int64_t t = 0; t < T; ++t) {
        if (slots[t] < 0) continue;
        int64_t blk = slots[t] / bs, off = slots[t] % bs;
        for (int h = 0; h < kvh; ++h) {
            const float *row = value + (t * kvh + h) * d;
            int64_t base = (blk * bs + off) * kvh + h;
            for (int gi = 0; gi < d / g; ++gi) {
                float mn = INFINITY, mx = -INFINITY;
                for (int i = 0; i < g; ++i) {
                    float x = row[gi * g + i];
                    if (x < mn) mn = x;
                    if (x > mx) mx = x;
                }
                float sc = group_scale(mn, mx);
                vs[base * (d / g) + gi] = sc;
                vm[base * (d / g) + gi] = mn;
                for (int w = 0; w < g / 8; ++w) {
                    uint32_t word = 0;
                    for (int lane = 0; lane < 8; ++lane)
                        word |= (uint32_t)quantize(row[gi * g + 8 * w + lane], mn, sc)
                                << (4 * lane);
                    vq[base * (d / 8) + (gi * g) / 8 + w] = (int32_t)word;
                }
            }
        }
    }
}

/* Gather-dequant: pkg/ops/kivi_gather.py:108-156.  Output fp32 [sum L, KVH, D]
 * (the caller casts); q*scale and +mn round separately. */
void ref_gather(const int32_t *kq, const float *ks, const float *km, const int32_t *vq,
                const float *vs, const float *vm, int bs, int kvh, int d, int g,
                const int64_t *block_table, int64_t batch, int64_t maxb,
                const int64_t *seq_lens, float *out_k, float *out_v) {
    int64_t row = 0;
    for (int64_t b = 0; b < batch; ++b) {
        for (int64_t p = 0; p < seq_lens[b]; ++p, ++row) {
            int64_t blk = block_table[b * maxb + p / bs];
            if (blk < 0) blk = 0;
            int64_t off = p % bs;
            for (int h = 0; h < kvh; ++h) {
                for (int c = 0; c < d; ++c) {
                    int64_t krow = (blk * kvh + h) * d + c;
                    uint32_t kw = (uint32_t)kq[krow * (bs / 8) + off / 8];
                    float kc = (float)((kw >> (4 * (off % 8))) & 0xF);
                    float kval = kc * ks[krow * (bs / g) + off / g];
                    kval = kval + km[krow * (bs / g) + off / g];
                    out_k[(row * kvh + h) * d + c] = kval;

                    int64_t vbase = (blk * bs + off) * kvh + h;
                    uint32_t vw = (uint32_t)vq[vbase * (d / 8) + c / 8];
                    float vc = (float)((vw >> (4 * (c % 8))) & 0xF);
                    float vval = vc * vs[vbase * (d / g) + c / g];
                    vval = vval + vm[vbase * (d / g) + c / g];
                    out_v[(row * kvh + h) * d + c] = vval;
                }
            }
        }
    }
}

/* bf16 round-to-nearest-even of an fp32 value (NaN not expected here). */
static float bf16_rne(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    u &= 0xFFFF0000u;
    float r;
    memcpy(&r, &u, 4);
    return r;
}

/* INT8 scales in bf16 arithmetic: i8ab.py:138-149 as torch evaluates it --
 * amax (exact), clamp_min(1e-12) -> bf16(1e-12), inv = bf16(bf16(1/amax)*127),
 * aq = bf16(1/inv).  x holds bf16 values widened to fp32, [T, C]. */
void ref_int8_scales_bf16(const float *x, int64_t T, int64_t C, float *inv, float *aq) {
    const float floor_val = bf16_rne(1.0e-12f);
    for (int64_t c = 0; c < C; ++c) {
        float a = 0.0f;
        for (int64_t t = 0; t < T; ++t) {
            float v = fabsf(x[t * C + c]);
            if (v > a) a = v;
        }
        if (a < 1.0e-12f) a = floor_val;
        float r = bf16_rne(1.0f / a);
        float i = bf16_rne(r * 127.0f);
        inv[c] = i;
        aq[c] = bf16_rne(1.0f / i);
    }
}

/* INT8 quantize in bf16: i8ab.py:161-170 -- bf16(x*inv), round half to even,
 * clamp to [-128, 127]. */
void ref_int8_quant_bf16(const float *x, int64_t T, int64_t C, const float *inv,
                         int8_t *out) {
    for (int64_t t = 0; t < T; ++t) {
        for (int64_t c = 0; c < C; ++c) {
            float p = bf16_rne(x[t * C + c] * inv[c]);
            float r = nearbyintf(p); /* default rounding mode: to nearest even */
            if (r < -128.0f) r = -128.0f;
            if (r > 127.0f) r = 127.0f;
            out[t * C + c] = (int8_t)r;
        }
    }
}
