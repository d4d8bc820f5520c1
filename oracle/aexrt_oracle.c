/*
 * aexrt_oracle.c -- CPU restatement of the AEXRT W8A8 convolution chain.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (aexrt_amd/, the C-ABI
 * library) links, loads or calls this file.  It is used by tests/, by the
 * smoke check in __graft_entry__.py and by the cpu_baseline leg of bench.py,
 * always as the checker and never as the thing measured or shipped.
 *
 * Every function restates one piece of the reference's algorithm and names
 * the reference file:line it follows ("RT" = native/aexrt_d3d12_runtime.cpp,
 * "ENG" = src/aexrt/engine.py).  Layouts follow the reference: activations
 * NCHW, weights [oc][ic][kh][kw].  Compile with -ffp-contract=off so that no
 * multiply-add is fused behind the restatement's back.
 *
 * Pinning status of each function is listed in the module docstring of
 * oracle/__init__.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------ */
/* fp16 <-> fp32 (IEEE binary16, round-to-nearest-even)               */
/* ------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

EXPORT float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0) {
        float v = (float)m * (1.0f / 16777216.0f); /* m * 2^-24, exact */
        return sign ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7F800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

EXPORT uint16_t or_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    x &= 0x7FFFFFFFu;
    if (x >= 0x7F800000u) return sign | (x > 0x7F800000u ? 0x7E00u : 0x7C00u);
    if (x >= 0x477FF000u) return sign | 0x7C00u;           /* >= 65520 -> inf */
    if (x < 0x38800000u) {                                 /* |f| < 2^-14 */
        float a = u2f(x) * 16777216.0f;                    /* exact scaling */
        return sign | (uint16_t)rintf(a);                  /* RNE, 1024 -> min normal */
    }
    uint32_t r = x - (112u << 23);
    r += 0xFFFu + ((r >> 13) & 1u);
    return sign | (uint16_t)(r >> 13);
}

EXPORT float or_round_f16(float f) { return or_f16_to_f32(or_f32_to_f16(f)); }

EXPORT void or_round_f16_array(float* x, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) x[i] = or_round_f16(x[i]);
}

/* ------------------------------------------------------------------ */
/* a1: amax zero + scan                                                */
/* ------------------------------------------------------------------ */

/* Per-tensor slot amax[0]: max |x| over every element of the tensor, all
 * batch images included (RT:3219-3259, the InterlockedMax into amax_out[0];
 * recorded over `elements` = N*C*H*W at RT:21631-21640).  Returned as the
 * float's bit pattern, which is how the reference stores it. */
EXPORT uint32_t or_amax_bits(const float* x, uint64_t n) {
    float m = 0.0f;
    for (uint64_t i = 0; i < n; ++i) {
        float a = fabsf(x[i]);
        if (a > m) m = a;
    }
    return f2u(m);
}

/* Full amax buffer as the reference fills it (RT:3219-3259): out[0] is the
 * per-tensor max; out[1+g] is the max over the contiguous memory strip
 * [g*16*plane, (g+1)*16*plane) with plane = elements/C = N*H*W.  For N == 1
 * the strip is channels 16g..16g+15; for N > 1 it is a memory strip, not a
 * per-sample channel group (the reference's behaviour, kept as is).
 * The zero pass (RT:3193-3199) is the initialisation to 0. */
EXPORT void or_amax_slots(const float* x, uint32_t N, uint32_t C, uint32_t HW,
                          uint32_t* out) {
    const uint64_t plane = (uint64_t)N * HW;
    const uint32_t g16 = C / 16u;
    float global = 0.0f;
    for (uint32_t g = 0; g < g16; ++g) {
        float m = 0.0f;
        const uint64_t b = (uint64_t)g * 16u * plane, e = b + 16u * plane;
        for (uint64_t i = b; i < e; ++i) {
            float a = fabsf(x[i]);
            if (a > m) m = a;
        }
        out[1 + g] = f2u(m);
        if (m > global) global = m;
    }
    /* The reference dispatches C/16 groups (RT:21631-21640), so memory past
     * the last full strip is never scanned when C % 16 != 0 (and amax stays
     * 0 when C < 16).  Restated as is; the product refuses int8 for such
     * inputs instead. */
    out[0] = f2u(global);
}

/* ------------------------------------------------------------------ */
/* a2: quantize / pack                                                 */
/* ------------------------------------------------------------------ */

/* D3D float->int conversion saturates (NaN -> 0); C's cast is undefined
 * out of range, so saturate explicitly before the low-byte wrap. */
static inline uint32_t q_byte(float v) {
    float r = rintf(v); /* HLSL round() == round-half-to-even */
    int32_t q;
    if (r != r) q = 0;
    else if (r >= 2147483647.0f) q = 2147483647;
    else if (r <= -2147483648.0f) q = (int32_t)0x80000000u;
    else q = (int32_t)r;
    return (uint32_t)q & 0xFFu;
}

/* Element quantizer of the pack pass (RT:3337-3344): s = 127/amax in fp32,
 * q = int(round(x * s)) & 0xFF; amax <= 0 packs zero. */
EXPORT int8_t or_quantize_value(float x, float amax) {
    if (!(amax > 0.0f)) return 0;
    const float s = 127.0f / amax;
    return (int8_t)(uint8_t)q_byte(x * s);
}

/* Layout-free form: q[i] for every element with one per-tensor amax. */
EXPORT void or_quantize(const float* x, uint64_t n, float amax, int8_t* q) {
    if (!(amax > 0.0f)) { memset(q, 0, n); return; }
    const float s = 127.0f / amax;
    for (uint64_t i = 0; i < n; ++i) q[i] = (int8_t)(uint8_t)q_byte(x[i] * s);
}

/* Reference packed layout (RT:3314-3346): packed[(n*C/4 + icg)*HW + pos]
 * holds channels 4icg..4icg+3 at one position, byte j = channel 4icg+j.
 * per_group selects amax[1 + icg/4] (RT:3330-3334, AEXRT_INT8_PACK_PERGROUP),
 * otherwise amax[0]. */
EXPORT void or_quant_pack(const float* x, uint32_t N, uint32_t C, uint32_t HW,
                          const uint32_t* amax, int per_group, uint32_t* packed) {
    const uint32_t icg_count = C / 4u;
    const uint64_t total4 = (uint64_t)N * icg_count * HW;
    for (uint64_t idx = 0; idx < total4; ++idx) {
        const uint32_t pos = (uint32_t)(idx % HW);
        const uint64_t t = idx / HW;
        const uint32_t icg = (uint32_t)(t % icg_count);
        const uint32_t n = (uint32_t)(t / icg_count);
        const float a = u2f(per_group ? amax[icg / 4u + 1u] : amax[0]);
        if (!(a > 0.0f)) { packed[idx] = 0u; continue; }
        const float s = 127.0f / a;
        const uint64_t base = ((uint64_t)n * icg_count + icg) * 4u * HW + pos;
        packed[idx] = q_byte(x[base] * s) | (q_byte(x[base + HW] * s) << 8) |
                      (q_byte(x[base + 2u * HW] * s) << 16) |
                      (q_byte(x[base + 3u * HW] * s) << 24);
    }
}

/* a3: fused amax+pack, pg16 (RT:4083-4149).  One pass per (n, 16-channel
 * group): the group max is taken over channels 16g..16g+15 of SAMPLE 0's
 * memory for every n (the shader's strip `begin` carries no n offset), the
 * slot amax[1+g] keeps the last writer, and the pack uses the n offset.
 * Restated as written; opt-in in the reference (ENABLE_QUANT_FUSED). */
EXPORT void or_quant_fused_pg16(const float* x, uint32_t N, uint32_t C, uint32_t HW,
                                uint32_t* packed, uint32_t* amax) {
    const uint32_t icg_count = C / 4u, g16_count = C / 16u;
    for (uint32_t n = 0; n < N; ++n) {
        for (uint32_t g = 0; g < g16_count; ++g) {
            float m = 0.0f;
            const uint64_t b = (uint64_t)g * 16u * HW, e = b + 16u * (uint64_t)HW;
            for (uint64_t i = b; i < e; ++i) { float a = fabsf(x[i]); if (a > m) m = a; }
            amax[g + 1u] = f2u(m);
            for (uint32_t il = 0; il < 4u; ++il) {
                const uint32_t icg = g * 4u + il;
                for (uint32_t pos = 0; pos < HW; ++pos) {
                    const uint64_t o = ((uint64_t)n * icg_count + icg) * HW + pos;
                    if (!(m > 0.0f)) { packed[o] = 0u; continue; }
                    const float s = 127.0f / m;
                    const uint64_t base = ((uint64_t)n * icg_count + icg) * 4u * HW + pos;
                    packed[o] = q_byte(x[base] * s) | (q_byte(x[base + HW] * s) << 8) |
                                (q_byte(x[base + 2u * HW] * s) << 16) |
                                (q_byte(x[base + 3u * HW] * s) << 24);
                }
            }
        }
    }
}

/* ------------------------------------------------------------------ */
/* a4: weight quantization, packed layout 8                            */
/* ------------------------------------------------------------------ */

/* ENG:2418-2465: per output channel scale = max|w|/127 (1 when the row is
 * all zero), inv = 1/scale in fp32, p = w*inv in fp32, q = clamp(sign(p) *
 * floor(|p| + 0.5), -127, 127) with |p| + 0.5 itself rounded to fp32 (the
 * compiler's numpy expression, ENG:2453-2456).  fp16 engines round the
 * source to fp16 first (ENG:2447-2448).  The runtime fallback for engines
 * without layout 8 (RT:21716-21741) uses std::round instead, which differs
 * only for |p| = 0.5 - 2^-25 (0 there, 1 here).
 * Layout 8 payload = q in [oc][ic][kk] order followed by oc fp32 scales. */
EXPORT void or_weight_quant(const float* w, uint32_t oc, uint32_t per_oc, int fp16_round,
                            int8_t* q, float* scale) {
    for (uint32_t o = 0; o < oc; ++o) {
        const float* row = w + (uint64_t)o * per_oc;
        float amax = 0.0f;
        for (uint32_t i = 0; i < per_oc; ++i) {
            float v = fp16_round ? or_round_f16(row[i]) : row[i];
            float a = fabsf(v);
            if (a > amax) amax = a;
        }
        const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
        const float inv = 1.0f / s;
        scale[o] = s;
        for (uint32_t i = 0; i < per_oc; ++i) {
            float v = fp16_round ? or_round_f16(row[i]) : row[i];
            float p = v * inv;
            float m = floorf(fabsf(p) + 0.5f);
            float r = p < 0.0f ? -m : (p > 0.0f ? m : 0.0f);
            if (r > 127.0f) r = 127.0f;
            if (r < -127.0f) r = -127.0f;
            q[(uint64_t)o * per_oc + i] = (int8_t)r;
        }
    }
}

/* ------------------------------------------------------------------ */
/* conv descriptor (yolo.py:929-939, aexrt.h AexrtConv2DDesc)          */
/* ------------------------------------------------------------------ */
typedef struct {
    uint32_t batch, in_c, in_h, in_w, out_c, out_h, out_w, kh, kw, sh, sw, pt, pl, dh, dw, groups;
} Desc;

static inline int in_bounds(int y, int x, const Desc* d) {
    return y >= 0 && y < (int)d->in_h && x >= 0 && x < (int)d->in_w;
}

/* ------------------------------------------------------------------ */
/* a5: int8 conv, per-tensor activation scale                          */
/* ------------------------------------------------------------------ */

/* int32 accumulator of the prequant conv (RT:4614-4762): acc = sum over
 * input channels and taps of q_a * q_w, zero padding, families 1x1 (s1 p0),
 * 3x3 s1 p1 and 3x3 s2 p1 (AEXRT_INT8_STRIDE2).  dot4add_i8packed is exact
 * integer arithmetic, so the loop order cannot change the result; the
 * general strides/pads of the descriptor are honoured.  qa: int8 NCHW,
 * qw: layout-8 int8 [oc][ic][kh*kw], acc: int32 NCHW. */
EXPORT void or_conv_int8_acc_mt(const int8_t* qa, const int8_t* qw, const uint32_t* desc,
                                int32_t* acc, int threads) {
    const Desc* d = (const Desc*)desc;
    const uint32_t kk = d->kh * d->kw;
    const int64_t jobs = (int64_t)d->batch * d->out_c;
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1) if (threads > 1)
    for (int64_t job = 0; job < jobs; ++job) {
    const uint32_t n = (uint32_t)(job / d->out_c), oc = (uint32_t)(job % d->out_c);
    for (uint32_t oy = 0; oy < d->out_h; ++oy)
    for (uint32_t ox = 0; ox < d->out_w; ++ox) {
        int32_t a = 0;
        for (uint32_t ic = 0; ic < d->in_c; ++ic)
        for (uint32_t ky = 0; ky < d->kh; ++ky) {
            const int iy = (int)(oy * d->sh + ky * d->dh) - (int)d->pt;
            for (uint32_t kx = 0; kx < d->kw; ++kx) {
                const int ix = (int)(ox * d->sw + kx * d->dw) - (int)d->pl;
                if (!in_bounds(iy, ix, d)) continue;
                const int32_t xa = qa[(((uint64_t)n * d->in_c + ic) * d->in_h + iy) * d->in_w + ix];
                const int32_t wv = qw[((uint64_t)oc * d->in_c + ic) * kk + ky * d->kw + kx];
                a += xa * wv;
            }
        }
        acc[(((uint64_t)n * d->out_c + oc) * d->out_h + oy) * d->out_w + ox] = a;
    }
    }
}

EXPORT void or_conv_int8_acc(const int8_t* qa, const int8_t* qw, const uint32_t* desc,
                             int32_t* acc) {
    or_conv_int8_acc_mt(qa, qw, desc, acc, 1);
}

static inline float silu(float v) { return v / (1.0f + expf(-v)); }

/* Dequant epilogue of the per-tensor prequant conv (RT:4669-4674 and
 * RT:4740-4745): in_scale = amax/127 (a separate fp32 division, not 1/s),
 * value = float(acc) * in_scale * w_scale[oc] + bias[oc], left to right,
 * then SiLU v / (1 + exp(-v)). */
EXPORT void or_conv_int8_epilogue(const int32_t* acc, uint32_t N, uint32_t OC, uint32_t HW,
                                  float amax, const float* w_scale, const float* bias,
                                  int do_silu, float* y) {
    const float in_scale = amax / 127.0f;
    for (uint64_t n = 0; n < N; ++n)
    for (uint32_t oc = 0; oc < OC; ++oc)
    for (uint32_t p = 0; p < HW; ++p) {
        const uint64_t i = (n * OC + oc) * HW + p;
        float v = (float)acc[i] * in_scale;
        v = v * w_scale[oc];
        v = v + bias[oc];
        y[i] = do_silu ? silu(v) : v;
    }
}

/* ------------------------------------------------------------------ */
/* a6: int8 conv with per-16-input-channel activation scales (pg16)    */
/* ------------------------------------------------------------------ */

static inline int32_t dot4(uint32_t a, uint32_t b, int32_t c) {
    for (int j = 0; j < 4; ++j)
        c += (int32_t)(int8_t)(a >> (8 * j)) * (int32_t)(int8_t)(b >> (8 * j));
    return c;
}

/* Pack helpers reproducing the reference's uint32 operands: activations
 * come from the NC/4HW4 pack, weights are layout-8 bytes gathered as
 * [oc][kk][icg] uint32 (RT:21744-21773). */
static inline uint32_t wpack(const int8_t* qw, const Desc* d, uint32_t oc, uint32_t icg,
                             uint32_t kidx, uint32_t kk) {
    uint32_t p = 0;
    for (uint32_t c = 0; c < 4u; ++c)
        p |= (uint32_t)(uint8_t)qw[((uint64_t)oc * d->in_c + icg * 4u + c) * kk + kidx] << (8u * c);
    return p;
}

static inline uint32_t apack_at(const uint32_t* pa, const Desc* d, uint32_t n, uint32_t icg,
                                int iy, int ix) {
    if (!in_bounds(iy, ix, d)) return 0u;
    const uint32_t icg_count = d->in_c / 4u;
    return pa[((uint64_t)n * icg_count + icg) * d->in_h * d->in_w + (uint64_t)iy * d->in_w + ix];
}

/* pg16 prequant conv (RT:4770-4923): int32 sub-sums over one 16-channel
 * group (2 icg per step for 1x1, 4 icg x 1 tap per step for 3x3), each
 * converted and scaled by amax[1+icg/4]/127 into an fp32 accumulator, then
 * value = fp * w_scale + bias and SiLU.  family: 1 = 1x1, 3 = 3x3 s1,
 * 32 = 3x3 s2. */
EXPORT void or_conv_int8_pg(const uint32_t* pa, const int8_t* qw, const uint32_t* desc,
                            uint32_t family, const uint32_t* amax, const float* w_scale,
                            const float* bias, int do_silu, float* y) {
    const Desc* d = (const Desc*)desc;
    const uint32_t icg_count = d->in_c / 4u;
    const uint32_t spatial = d->out_h * d->out_w;
    const uint32_t kk = family == 1u ? 1u : 9u;
    const uint32_t stride = family == 32u ? 2u : 1u;
    for (uint32_t n = 0; n < d->batch; ++n)
    for (uint32_t oc = 0; oc < d->out_c; ++oc)
    for (uint32_t pos = 0; pos < spatial; ++pos) {
        const uint32_t oh = pos / d->out_w, ow = pos % d->out_w;
        float fp = 0.0f;
        if (family == 1u) {
            uint32_t icg = 0;
            for (; icg + 2u <= icg_count; icg += 2u) {
                const float g = u2f(amax[icg / 4u + 1u]) / 127.0f;
                const uint32_t a0 = apack_at(pa, d, n, icg, (int)oh, (int)ow);
                const uint32_t a1 = apack_at(pa, d, n, icg + 1u, (int)oh, (int)ow);
                int32_t s = dot4(a1, wpack(qw, d, oc, icg + 1u, 0, 1),
                                 dot4(a0, wpack(qw, d, oc, icg, 0, 1), 0));
                fp += (float)s * g;
            }
            for (; icg < icg_count; ++icg) {
                const float g = u2f(amax[icg / 4u + 1u]) / 127.0f;
                const uint32_t a = apack_at(pa, d, n, icg, (int)oh, (int)ow);
                fp += (float)dot4(a, wpack(qw, d, oc, icg, 0, 1), 0) * g;
            }
        } else {
            uint32_t icg = 0;
            for (; icg + 4u <= icg_count; icg += 4u) {
                const float g = u2f(amax[icg / 4u + 1u]) / 127.0f;
                for (uint32_t k = 0; k < 9u; ++k) {
                    const int iy = (int)(oh * stride + k / 3u) - 1;
                    const int ix = (int)(ow * stride + k % 3u) - 1;
                    int32_t s = 0;
                    for (uint32_t q = 0; q < 4u; ++q)
                        s = dot4(apack_at(pa, d, n, icg + q, iy, ix),
                                 wpack(qw, d, oc, icg + q, k, kk), s);
                    fp += (float)s * g;
                }
            }
            for (; icg < icg_count; ++icg) {
                const float g = u2f(amax[icg / 4u + 1u]) / 127.0f;
                for (uint32_t k = 0; k < 9u; ++k) {
                    const int iy = (int)(oh * stride + k / 3u) - 1;
                    const int ix = (int)(ow * stride + k % 3u) - 1;
                    fp += (float)dot4(apack_at(pa, d, n, icg, iy, ix),
                                      wpack(qw, d, oc, icg, k, kk), 0) * g;
                }
            }
        }
        float v = fp * w_scale[oc];
        v = v + bias[oc];
        y[((uint64_t)n * d->out_c + oc) * spatial + pos] = do_silu ? silu(v) : v;
    }
}

/* ------------------------------------------------------------------ */
/* a8: K-split (4 slices) partial + combine                            */
/* ------------------------------------------------------------------ */

/* Per-tensor K-split (RT:3852-4010 non-PERGROUP branch, RT:4516-4544):
 * slice k covers icg [k*ips, min((k+1)*ips, icg_count)), ips =
 * ceil(icg_count/k_splits); partial = float(int32 slice sum) * in_scale *
 * w_scale[oc]; combine = bias + sum of partials in slice order, SiLU.
 * pg16 (per_group != 0): per-4-icg float accumulation with the group
 * scale of the step's first icg, times w_scale (RT:3880-3935). */
EXPORT void or_conv_int8_ksplit(const uint32_t* pa, const int8_t* qw, const uint32_t* desc,
                                uint32_t family, const uint32_t* amax, int per_group,
                                uint32_t k_splits, const float* w_scale, const float* bias,
                                int do_silu, float* y) {
    const Desc* d = (const Desc*)desc;
    const uint32_t icg_count = d->in_c / 4u;
    const uint32_t ips = (icg_count + k_splits - 1u) / k_splits;
    const uint32_t taps = family == 1u ? 1u : 9u;
    const uint32_t stride = d->sh;
    const uint32_t pad = d->pt;
    const uint32_t spatial = d->out_h * d->out_w;
    const float in_scale = u2f(amax[0]) / 127.0f;
    for (uint32_t n = 0; n < d->batch; ++n)
    for (uint32_t oc = 0; oc < d->out_c; ++oc)
    for (uint32_t pos = 0; pos < spatial; ++pos) {
        const uint32_t oh = pos / d->out_w, ow = pos % d->out_w;
        float sum = bias[oc];
        for (uint32_t ks = 0; ks < k_splits; ++ks) {
            const uint32_t b = ks * ips;
            const uint32_t e = b + ips < icg_count ? b + ips : icg_count;
            float part;
            if (!per_group) {
                int32_t s = 0;
                for (uint32_t icg = b; icg < e; ++icg)
                    for (uint32_t k = 0; k < taps; ++k) {
                        const int iy = (int)(oh * stride + (taps == 1u ? 0u : k / 3u)) - (int)pad;
                        const int ix = (int)(ow * stride + (taps == 1u ? 0u : k % 3u)) - (int)pad;
                        s = dot4(apack_at(pa, d, n, icg, iy, ix), wpack(qw, d, oc, icg, k, taps), s);
                    }
                part = (float)s * in_scale;
                part = part * w_scale[oc];
            } else {
                float fp = 0.0f;
                uint32_t icg = b;
                for (; icg + 4u <= e; icg += 4u) {
                    const float g = u2f(amax[icg / 4u + 1u]) / 127.0f;
                    for (uint32_t k = 0; k < taps; ++k) {
                        const int iy = (int)(oh * stride + (taps == 1u ? 0u : k / 3u)) - (int)pad;
                        const int ix = (int)(ow * stride + (taps == 1u ? 0u : k % 3u)) - (int)pad;
                        int32_t s = 0;
                        for (uint32_t q = 0; q < 4u; ++q)
                            s = dot4(apack_at(pa, d, n, icg + q, iy, ix),
                                     wpack(qw, d, oc, icg + q, k, taps), s);
                        fp += (float)s * g;
                    }
                }
                for (; icg < e; ++icg) {
                    const float g = u2f(amax[icg / 4u + 1u]) / 127.0f;
                    for (uint32_t k = 0; k < taps; ++k) {
                        const int iy = (int)(oh * stride + (taps == 1u ? 0u : k / 3u)) - (int)pad;
                        const int ix = (int)(ow * stride + (taps == 1u ? 0u : k % 3u)) - (int)pad;
                        fp += (float)dot4(apack_at(pa, d, n, icg, iy, ix),
                                          wpack(qw, d, oc, icg, k, taps), 0) * g;
                    }
                }
                part = fp * w_scale[oc];
            }
            sum += part;
        }
        y[((uint64_t)n * d->out_c + oc) * spatial + pos] = do_silu ? silu(sum) : sum;
    }
}

/* ------------------------------------------------------------------ */
/* a9: dynamic int8 fallback (in-kernel quantization)                  */
/* ------------------------------------------------------------------ */

/* RT:2952-3115.  1x1: each (position, 4-channel group) gets its own scale
 * s = 127/amax4 (0 when amax4 == 0) and dequant amax4/127; 3x3: the 36
 * values of one 4-channel group over the 9 taps share one scale, the taps
 * chain in int32 and the group is dequantized once.  acc (fp32) * w_scale
 * + bias, SiLU.  x: fp32 NCHW. */
EXPORT void or_conv_int8_dynamic(const float* x, const int8_t* qw, const uint32_t* desc,
                                 uint32_t family, const float* w_scale, const float* bias,
                                 int do_silu, float* y) {
    const Desc* d = (const Desc*)desc;
    const uint32_t icg_count = d->in_c / 4u;
    const uint32_t spatial = d->out_h * d->out_w;
    const uint32_t stride = family == 32u ? 2u : 1u;
    for (uint32_t n = 0; n < d->batch; ++n)
    for (uint32_t oc = 0; oc < d->out_c; ++oc)
    for (uint32_t pos = 0; pos < spatial; ++pos) {
        const uint32_t oh = pos / d->out_w, ow = pos % d->out_w;
        float acc = 0.0f;
        for (uint32_t icg = 0; icg < icg_count; ++icg) {
            const uint32_t ic = icg * 4u;
            if (family == 1u) {
                float v[4], am = 0.0f;
                for (uint32_t c = 0; c < 4u; ++c) {
                    v[c] = x[(((uint64_t)n * d->in_c + ic + c) * d->in_h + oh) * d->in_w + ow];
                    float a = fabsf(v[c]); if (a > am) am = a;
                }
                const float s = am > 0.0f ? 127.0f / am : 0.0f;
                const float inv = am / 127.0f;
                uint32_t a = q_byte(v[0] * s) | (q_byte(v[1] * s) << 8) |
                             (q_byte(v[2] * s) << 16) | (q_byte(v[3] * s) << 24);
                acc += (float)dot4(a, wpack(qw, d, oc, icg, 0, 1), 0) * inv;
            } else {
                float v[9][4], am = 0.0f;
                for (uint32_t k = 0; k < 9u; ++k) {
                    const int iy = (int)(oh * stride + k / 3u) - 1;
                    const int ix = (int)(ow * stride + k % 3u) - 1;
                    for (uint32_t c = 0; c < 4u; ++c) {
                        float val = 0.0f;
                        if (in_bounds(iy, ix, d))
                            val = x[(((uint64_t)n * d->in_c + ic + c) * d->in_h + iy) * d->in_w + ix];
                        v[k][c] = val;
                        float a = fabsf(val); if (a > am) am = a;
                    }
                }
                const float s = am > 0.0f ? 127.0f / am : 0.0f;
                const float inv = am / 127.0f;
                int32_t part = 0;
                for (uint32_t k = 0; k < 9u; ++k) {
                    uint32_t a = q_byte(v[k][0] * s) | (q_byte(v[k][1] * s) << 8) |
                                 (q_byte(v[k][2] * s) << 16) | (q_byte(v[k][3] * s) << 24);
                    part = dot4(a, wpack(qw, d, oc, icg, k, 9u), part);
                }
                acc += (float)part * inv;
            }
        }
        float v = acc * w_scale[oc];
        v = v + bias[oc];
        y[((uint64_t)n * d->out_c + oc) * spatial + pos] = do_silu ? silu(v) : v;
    }
}

/* ------------------------------------------------------------------ */
/* a15: the reference's CPU conv                                       */
/* ------------------------------------------------------------------ */

/* cpu_conv2d (RT:20552-20580): acc starts at bias, sums x*w over
 * (icg, ky, kx) of the group, skipping out-of-range taps; SiLU
 * acc / (1 + exp(-acc)).  Single thread unless threads > 1, in which case
 * the (n, oc) loop is split across OpenMP threads (each output is still
 * computed by the same ordered loop, so results do not depend on it). */
EXPORT void or_cpu_conv2d(const float* x, const float* w, const float* b, float* y,
                          const uint32_t* desc, int do_silu, int threads) {
    const Desc* d = (const Desc*)desc;
    const uint32_t ocpg = d->out_c / d->groups, icpg = d->in_c / d->groups;
    const int64_t jobs = (int64_t)d->batch * d->out_c;
    (void)threads;
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1) if (threads > 1)
    for (int64_t job = 0; job < jobs; ++job) {
        const uint32_t n = (uint32_t)(job / d->out_c), oc = (uint32_t)(job % d->out_c);
        const uint32_t gid = oc / ocpg;
        for (uint32_t oy = 0; oy < d->out_h; ++oy)
        for (uint32_t ox = 0; ox < d->out_w; ++ox) {
            float acc = b[oc];
            for (uint32_t icg = 0; icg < icpg; ++icg) {
                const uint32_t ic = gid * icpg + icg;
                for (uint32_t ky = 0; ky < d->kh; ++ky) {
                    const int iy = (int)(oy * d->sh + ky * d->dh) - (int)d->pt;
                    if (iy < 0 || iy >= (int)d->in_h) continue;
                    for (uint32_t kx = 0; kx < d->kw; ++kx) {
                        const int ix = (int)(ox * d->sw + kx * d->dw) - (int)d->pl;
                        if (ix < 0 || ix >= (int)d->in_w) continue;
                        const uint64_t xi = (((uint64_t)n * d->in_c + ic) * d->in_h + iy) * d->in_w + ix;
                        const uint64_t wi = (((uint64_t)oc * icpg + icg) * d->kh + ky) * d->kw + kx;
                        acc += x[xi] * w[wi];
                    }
                }
            }
            if (do_silu) acc = acc / (1.0f + expf(-acc));
            y[(((uint64_t)n * d->out_c + oc) * d->out_h + oy) * d->out_w + ox] = acc;
        }
    }
}

/* ------------------------------------------------------------------ */
/* a12: Winograd F(2x2,3x3)                                            */
/* ------------------------------------------------------------------ */

/* Weight transform U = G g G^T, G = [[1,0,0],[.5,.5,.5],[.5,-.5,.5],[0,0,1]]
 * on the fp16-rounded source (ENG:2346-2415), layout [oc][ic][4][4].
 * Evaluated as T = g G^T then U = G T, each dot product in fp32 in index
 * order; to_f16 != 0 rounds the result to fp16 (layout 3), else fp32
 * (layout 5). */
EXPORT void or_winograd_f2x2_weight(const float* w, uint32_t oc, uint32_t ic, int to_f16,
                                    float* u) {
    static const float G[4][3] = {{1.f, 0.f, 0.f}, {.5f, .5f, .5f}, {.5f, -.5f, .5f}, {0.f, 0.f, 1.f}};
    const uint64_t count = (uint64_t)oc * ic;
    for (uint64_t p = 0; p < count; ++p) {
        float g[3][3], t[3][4];
        for (int i = 0; i < 9; ++i) g[i / 3][i % 3] = or_round_f16(w[p * 9 + i]);
        for (int k = 0; k < 3; ++k)
            for (int bb = 0; bb < 4; ++bb) {
                float s = 0.0f;
                for (int l = 0; l < 3; ++l) s += g[k][l] * G[bb][l];
                t[k][bb] = s;
            }
        for (int a = 0; a < 4; ++a)
            for (int bb = 0; bb < 4; ++bb) {
                float s = 0.0f;
                for (int k = 0; k < 3; ++k) s += G[a][k] * t[k][bb];
                u[p * 16 + a * 4 + bb] = to_f16 ? or_round_f16(s) : s;
            }
    }
}

/* Winograd conv with fp32 accumulation (RT:2480-2631, kernel 46 = the
 * AEXRT_FP32_ACCUM build): per 2x2 output tile, d = 4x4 input patch at
 * (2ty-1, 2tx-1) with zero padding; rows t_i = (d0-d2, d1+d2, -d1+d2, d1-d3)
 * (RT:2533-2548); v0 = t0-t2, v1 = t1+t2, v2 = -t1+t2, v3 = t1-t3; m_r +=
 * v_r * U_r over ic, summed in 8-channel partials (RT:2585-2608); output
 * r0 = m0+m1+m2, r1 = m1-m2-m3, (r0.x+r0.y+r0.z, r0.y-r0.z-r0.w,
 * r1.x+r1.y+r1.z, r1.y-r1.z-r1.w) + bias, SiLU as v * (1/(1+exp(-v)))
 * (RT:2612-2628).  Requires 3x3 s1 p1 and even out_h/out_w. */
EXPORT void or_winograd_f2x2_conv(const float* x, const float* u, const float* bias,
                                  const uint32_t* desc, float* y) {
    const Desc* d = (const Desc*)desc;
    const uint32_t tiles_w = d->out_w / 2u, tiles_h = d->out_h / 2u;
    const uint32_t C = d->in_c;
    float* vt = (float*)malloc(sizeof(float) * 16u * C);
    for (uint32_t n = 0; n < d->batch; ++n)
    for (uint32_t ty = 0; ty < tiles_h; ++ty)
    for (uint32_t tx = 0; tx < tiles_w; ++tx) {
        const int y0 = (int)(ty * 2u) - 1, x0 = (int)(tx * 2u) - 1;
        for (uint32_t c = 0; c < C; ++c) {
            float dd[4][4], t[4][4];
            for (int r = 0; r < 4; ++r)
                for (int q = 0; q < 4; ++q) {
                    const int iy = y0 + r, ix = x0 + q;
                    dd[r][q] = in_bounds(iy, ix, d)
                        ? x[(((uint64_t)n * C + c) * d->in_h + iy) * d->in_w + ix] : 0.0f;
                }
            for (int r = 0; r < 4; ++r) {
                t[r][0] = dd[r][0] - dd[r][2];
                t[r][1] = dd[r][1] + dd[r][2];
                t[r][2] = -dd[r][1] + dd[r][2];
                t[r][3] = dd[r][1] - dd[r][3];
            }
            for (int q = 0; q < 4; ++q) {
                vt[c * 16u + 0 * 4 + q] = t[0][q] - t[2][q];
                vt[c * 16u + 1 * 4 + q] = t[1][q] + t[2][q];
                vt[c * 16u + 2 * 4 + q] = -t[1][q] + t[2][q];
                vt[c * 16u + 3 * 4 + q] = t[1][q] - t[3][q];
            }
        }
        for (uint32_t oc = 0; oc < d->out_c; ++oc) {
            float m[4][4] = {{0}};
            for (uint32_t base = 0; base < C; base += 8u) {
                float part[4][4] = {{0}};
                for (uint32_t l = 0; l < 8u && base + l < C; ++l) {
                    const uint32_t c = base + l;
                    const float* uu = u + ((uint64_t)oc * C + c) * 16u;
                    for (int r = 0; r < 4; ++r)
                        for (int q = 0; q < 4; ++q)
                            part[r][q] += vt[c * 16u + r * 4 + q] * uu[r * 4 + q];
                }
                for (int r = 0; r < 4; ++r)
                    for (int q = 0; q < 4; ++q) m[r][q] += part[r][q];
            }
            float r0[4], r1[4], res[4];
            for (int q = 0; q < 4; ++q) {
                r0[q] = m[0][q] + m[1][q] + m[2][q];
                r1[q] = m[1][q] - m[2][q] - m[3][q];
            }
            res[0] = r0[0] + r0[1] + r0[2];
            res[1] = r0[1] - r0[2] - r0[3];
            res[2] = r1[0] + r1[1] + r1[2];
            res[3] = r1[1] - r1[2] - r1[3];
            const uint64_t ob = ((uint64_t)n * d->out_c + oc) * d->out_h * d->out_w;
            const uint32_t oy = ty * 2u, ox = tx * 2u;
            for (int q = 0; q < 4; ++q) {
                float v = res[q] + bias[oc];
                v = v * (1.0f / (1.0f + expf(-v)));
                res[q] = v;
            }
            y[ob + oy * d->out_w + ox] = res[0];
            y[ob + oy * d->out_w + ox + 1] = res[1];
            y[ob + (oy + 1) * d->out_w + ox] = res[2];
            y[ob + (oy + 1) * d->out_w + ox + 1] = res[3];
        }
    }
    free(vt);
}

/* ------------------------------------------------------------------ */
/* Glue ops of the replay stream used by the network oracle            */
/* ------------------------------------------------------------------ */

/* MAXPOOL (yolo.py:862-871 params; cpu_maxpool semantics: out-of-range
 * taps are skipped, max over the window). */
EXPORT void or_maxpool(const float* x, uint32_t N, uint32_t C, uint32_t H, uint32_t W,
                       uint32_t k, uint32_t s, uint32_t p, float* y, uint32_t OH, uint32_t OW) {
    for (uint64_t nc = 0; nc < (uint64_t)N * C; ++nc)
    for (uint32_t oy = 0; oy < OH; ++oy)
    for (uint32_t ox = 0; ox < OW; ++ox) {
        float m = -INFINITY;
        for (uint32_t ky = 0; ky < k; ++ky) {
            const int iy = (int)(oy * s + ky) - (int)p;
            if (iy < 0 || iy >= (int)H) continue;
            for (uint32_t kx = 0; kx < k; ++kx) {
                const int ix = (int)(ox * s + kx) - (int)p;
                if (ix < 0 || ix >= (int)W) continue;
                const float v = x[(nc * H + iy) * W + ix];
                if (v > m) m = v;
            }
        }
        y[(nc * OH + oy) * OW + ox] = m;
    }
}

/* RESIZE nearest (yolo.py:855-859 params): source index = dst * in / out. */
EXPORT void or_resize_nearest(const float* x, uint32_t N, uint32_t C, uint32_t H, uint32_t W,
                              float* y, uint32_t OH, uint32_t OW) {
    for (uint64_t nc = 0; nc < (uint64_t)N * C; ++nc)
    for (uint32_t oy = 0; oy < OH; ++oy)
    for (uint32_t ox = 0; ox < OW; ++ox) {
        const uint32_t iy = (uint32_t)((uint64_t)oy * H / OH);
        const uint32_t ix = (uint32_t)((uint64_t)ox * W / OW);
        y[(nc * OH + oy) * OW + ox] = x[(nc * H + iy) * W + ix];
    }
}

/* ------------------------------------------------------------------ */
/* YOLO postprocess of output0 (the reference's GPU path)              */
/* ------------------------------------------------------------------ */

static float yolo_iou(const float* a, const float* b) {
    const float x1 = fmaxf(a[0], b[0]), y1 = fmaxf(a[1], b[1]);
    const float x2 = fminf(a[2], b[2]), y2 = fminf(a[3], b[3]);
    const float iw = fmaxf(0.0f, x2 - x1), ih = fmaxf(0.0f, y2 - y1);
    const float inter = iw * ih;
    const float area_a = fmaxf(0.0f, a[2] - a[0]) * fmaxf(0.0f, a[3] - a[1]);
    const float area_b = fmaxf(0.0f, b[2] - b[0]) * fmaxf(0.0f, b[3] - b[1]);
    return inter / fmaxf(area_a + area_b - inter, 1e-7f);
}

static int yolo_outranks(float sj, uint32_t j, float si, uint32_t i) { return sj > si || (sj == si && j < i); }

/* NMS mark (RT:15637-15691) and top-k (RT:15693-15735) over count
 * candidates: a candidate is dropped when a candidate of the same class
 * that outranks it (higher score, or equal score and lower index) has
 * IoU > iou with it -- every such candidate counts, suppressed or not
 * (unlike greedy NMS); a kept candidate's rank among the kept ones is its
 * output slot; returns min(kept, max_det). */
static uint32_t yolo_nms_topk(const float* cand, uint32_t count, float iou, uint32_t max_det,
                              uint32_t* keep, float* dets) {
    for (uint32_t i = 0; i < count; ++i) {
        keep[i] = 1u;
        for (uint32_t j = 0; j < count; ++j) {
            if (j == i || cand[6u * j + 5u] != cand[6u * i + 5u]) continue;
            if (yolo_outranks(cand[6u * j + 4u], j, cand[6u * i + 4u], i) &&
                yolo_iou(cand + 6u * i, cand + 6u * j) > iou) { keep[i] = 0u; break; }
        }
    }
    uint32_t kept = 0;
    for (uint32_t i = 0; i < count; ++i) {
        if (!keep[i]) continue;
        ++kept;
        uint32_t rank = 0;
        for (uint32_t j = 0; j < count; ++j)
            if (j != i && keep[j] && yolo_outranks(cand[6u * j + 4u], j, cand[6u * i + 4u], i)) ++rank;
        if (rank < max_det) memcpy(dets + 6u * rank, cand + 6u * i, 6u * sizeof(float));
    }
    return kept < max_det ? kept : max_det;
}

/* decode/filter of a decoded output0 (RT:15300-15356): per anchor the best
 * class score times objectness (strict >: first max wins), kept unless
 * score < conf, box cx -/+ 0.5 w; the reference appends with an atomic
 * counter, restated here in anchor order (one order it can produce) and
 * capped at max_cand.  layout 2: out[a * channels + ch], else
 * out[ch * anchors + a].  cand: scratch of max_cand * 6 floats, keep:
 * max_cand words. */
EXPORT uint32_t or_yolo_decode_nms_topk(const float* out, uint32_t layout, uint32_t anchors,
                                        uint32_t channels, uint32_t classes, uint32_t has_obj,
                                        float conf, float iou, uint32_t max_cand, uint32_t max_det,
                                        float* cand, uint32_t* keep, float* dets) {
#define RD(ch, a) (layout == 2u ? out[(uint64_t)(a) * channels + (ch)] : out[(uint64_t)(ch) * anchors + (a)])
    const uint32_t cls_off = has_obj ? 5u : 4u;
    uint32_t total = 0;
    for (uint32_t a = 0; a < anchors && classes > 0; ++a) {
        const float obj = has_obj ? RD(4u, a) : 1.0f;
        float best = obj * RD(cls_off, a);
        uint32_t best_cls = 0;
        for (uint32_t c = 1; c < classes; ++c) {
            const float s = obj * RD(cls_off + c, a);
            if (s > best) { best = s; best_cls = c; }
        }
        if (best < conf) continue;
        const uint32_t idx = total++;
        if (idx >= max_cand) continue;
        const float cx = RD(0u, a), cy = RD(1u, a), w = RD(2u, a), h = RD(3u, a);
        const float hw = 0.5f * w, hh = 0.5f * h;
        float* c = cand + 6u * idx;
        c[0] = cx - hw; c[1] = cy - hh; c[2] = cx + hw; c[3] = cy + hh;
        c[4] = best; c[5] = (float)best_cls;
    }
#undef RD
    return yolo_nms_topk(cand, total < max_cand ? total : max_cand, iou, max_det, keep, dets);
}

/* e^x of the postprocess: Cody-Waite reduction x = k ln2 + r (ln2 as a
 * 16-bit head, so k * head is exact, plus a tail), |r| <= ln2/2, e^r by
 * the degree-7 Taylor polynomial in Horner form, times 2^k; 0 below -87,
 * infinity above 88.5.  The product kernel computes the same operations
 * (the reference's exp belongs to its shader compiler and driver). */
EXPORT float or_post_exp(float x) {
    if (x != x) return x;
    if (x < -87.0f) return 0.0f;
    if (x > 88.5f) return INFINITY;
    const float k = rintf(x * 1.44269504f);
    const float r = (x - k * 0.693145751953125f) - k * 1.42860677e-06f;
    float p = 1.0f / 5040.0f;
    p = p * r + 1.0f / 720.0f;
    p = p * r + 1.0f / 120.0f;
    p = p * r + 1.0f / 24.0f;
    p = p * r + 1.0f / 6.0f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    return ldexpf(p, (int)k);
}

/* Raw Detect head (the post-conv part of RT:15465-15636): head[ch][a]
 * (layout 2: [a][ch]) with channels 0..63 the 4 x 16 DFL bin logits and
 * 64.. the class logits; score = 1 / (1 + exp(-logit)), best class strict
 * >; kept unless score < conf; side d = sum_b e_b b / max(sum_b e_b,
 * 1e-20), e_b = exp(l_b - max_b l_b); anchors level by level (lev_hw[2l] x
 * lev_hw[2l+1], stride lev_stride[l]), centre (gx + 0.5, gy + 0.5), box =
 * ((ax - d0) s, (ay - d1) s, (ax + d2) s, (ay + d3) s). */
EXPORT uint32_t or_yolo_dfl_decode_nms_topk(const float* head, uint32_t layout, uint32_t nlev,
                                            const uint32_t* lev_hw, const float* lev_stride,
                                            uint32_t classes, float conf, float iou, uint32_t max_cand,
                                            uint32_t max_det, float* cand, uint32_t* keep, float* dets) {
    uint32_t anchors = 0;
    for (uint32_t l = 0; l < nlev; ++l) anchors += lev_hw[2u * l] * lev_hw[2u * l + 1u];
    const uint32_t channels = 64u + classes;
#define RD(ch, a) (layout == 2u ? head[(uint64_t)(a) * channels + (ch)] : head[(uint64_t)(ch) * anchors + (a)])
    uint32_t total = 0, a = 0;
    for (uint32_t l = 0; l < nlev; ++l) {
        const uint32_t gh = lev_hw[2u * l], gw = lev_hw[2u * l + 1u];
        for (uint32_t pos = 0; pos < gh * gw; ++pos, ++a) {
            float best = 1.0f / (1.0f + or_post_exp(-RD(64u, a)));
            uint32_t best_cls = 0;
            for (uint32_t c = 1; c < classes; ++c) {
                const float s = 1.0f / (1.0f + or_post_exp(-RD(64u + c, a)));
                if (s > best) { best = s; best_cls = c; }
            }
            if (best < conf) continue;
            const uint32_t idx = total++;
            if (idx >= max_cand) continue;
            float dist[4];
            for (uint32_t d = 0; d < 4u; ++d) {
                float m = -3.402823e38f;
                for (uint32_t b = 0; b < 16u; ++b) m = fmaxf(m, RD(16u * d + b, a));
                float sum = 0.0f, acc = 0.0f;
                for (uint32_t b = 0; b < 16u; ++b) {
                    const float e = or_post_exp(RD(16u * d + b, a) - m);
                    sum = sum + e;
                    acc = acc + e * (float)b;
                }
                dist[d] = acc / fmaxf(sum, 1e-20f);
            }
            const float ax = (float)(pos % gw) + 0.5f, ay = (float)(pos / gw) + 0.5f, s = lev_stride[l];
            float* c = cand + 6u * idx;
            c[0] = (ax - dist[0]) * s; c[1] = (ay - dist[1]) * s;
            c[2] = (ax + dist[2]) * s; c[3] = (ay + dist[3]) * s;
            c[4] = best; c[5] = (float)best_cls;
        }
    }
#undef RD
    return yolo_nms_topk(cand, total < max_cand ? total : max_cand, iou, max_det, keep, dets);
}
