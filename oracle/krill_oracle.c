/*
 * krill_oracle.c -- CPU restatement of Krill's int8 KV-cache hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or, for the baseline, as the thing timed beside the GPU).  The product
 * library (krill_amd/libkrillhip.so) never links, loads or calls it.
 *
 * Every function names the reference file:line it restates (paths are relative
 * to the srvsngh99/Krill source tree).  The reference is Swift on mlx-swift
 * 0.31.4 (a remote SwiftPM dependency, Package.swift:25); neither Swift nor
 * MLX exists here, so nothing of the reference is compiled or run: the
 * algorithm is restated from the source text.
 *
 * Pinning (how each function is checked independently of itself) is listed in
 * the header of oracle/oracle.py.  The exact rounding of MLX's fused SDPA
 * (third-party mlx) is the one boundary the oracle does not reproduce: the
 * attention checks are against binary64 within a stated tolerance.
 *
 * Build: gcc -O2 -std=c11 -fPIC -shared -ffp-contract=off -fno-fast-math -fopenmp
 * (-ffp-contract=off: no fused multiply-add may change a rounding step.)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* IEEE binary16 / bfloat16 <-> binary32, round-to-nearest-even.             */
/* ------------------------------------------------------------------------ */

static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24 is exact in binary32 */
        float f = (float)m * 5.9604644775390625e-08f;
        return bits_f32(f32_bits(f) | sign);
    }
    if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t oracle_f32_to_f16(float f) {
    uint32_t x = f32_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf / nan (nan keeps a quiet payload bit) */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u | ((ax >> 13) & 0x3ffu) : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                                   /* below 2^-14: subnormal */
        uint32_t e = ax >> 23;
        if (e < 102) return (uint16_t)sign;                   /* < 2^-25 -> +-0 */
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e;                            /* 14..24 */
        uint32_t r = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = (((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

float oracle_bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

uint16_t oracle_f32_to_bf16(float f) {
    uint32_t x = f32_bits(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

/* dtype tags shared with include/libkrillhip.h */
enum { DT_F16 = 0, DT_BF16 = 1 };

static inline float dt_to_f32(uint16_t v, int dt) {
    return dt == DT_BF16 ? oracle_bf16_to_f32(v) : oracle_f16_to_f32(v);
}
/* Round a binary32 value to the element dtype and back.  A binary16/bfloat16
 * add, sub, mul or div computed in binary32 and rounded once gives the
 * correctly rounded dtype result (24 >= 2*11+2), which is what MLX's CPU
 * kernels produce for these dtypes. */
static inline float dt_round(float f, int dt) {
    return dt == DT_BF16 ? oracle_bf16_to_f32(oracle_f32_to_bf16(f))
                         : oracle_f16_to_f32(oracle_f32_to_f16(f));
}

/* ------------------------------------------------------------------------ */
/* a1: QuantizedKVCache.quantizePerHead                                      */
/*     Sources/KrillCache/QuantizedKVCache.swift:181-197                     */
/* ------------------------------------------------------------------------ */
/*
 * Per row of `D` elements (one (batch, head, token)):
 *   mn = min(x), mx = max(x)                                 (:183-184, exact)
 *   scale = f32(round_dt(mx - mn)) / 255.0f                  (:185, dtype sub,
 *                                                             f32 promotion by
 *                                                             the Float array)
 *   safe  = max(scale, 1e-8f)                                (:187)
 *   n = f32(round_dt(x - mn)) / safe                         (:192)
 *   q = uint8(trunc(clip(n, 0, 255)))                        (:193-194)
 *   returns (q, f16(safe), f16(mn))                          (:196)
 *   (a zero mn is returned as +0: see below)
 */
void oracle_quantize_ref_rows(const uint16_t *x, int dt, int64_t n_rows, int D,
                              uint8_t *q, uint16_t *scale_f16, uint16_t *zero_f16) {
    for (int64_t r = 0; r < n_rows; ++r) {
        const uint16_t *xr = x + r * D;
        float mn = dt_to_f32(xr[0], dt), mx = mn;
        for (int d = 1; d < D; ++d) {
            float v = dt_to_f32(xr[d], dt);
            if (v < mn) mn = v;
            if (v > mx) mx = v;
        }
        float scale = dt_round(mx - mn, dt) / 255.0f;
        float safe = scale > 1e-8f ? scale : 1e-8f;
        for (int d = 0; d < D; ++d) {
            float n = dt_round(dt_to_f32(xr[d], dt) - mn, dt) / safe;
            if (n < 0.0f) n = 0.0f;
            if (n > 255.0f) n = 255.0f;
            q[r * D + d] = (uint8_t)n;
        }
        scale_f16[r] = oracle_f32_to_f16(safe);
        /* identity for f16 input, RNE for bf16; a zero minimum is stored as +0:
         * which of +0 / -0 a minimum over both returns depends on the order
         * of the comparisons (the kernels reduce in a tree) */
        zero_f16[r] = oracle_f32_to_f16(mn + 0.0f);
    }
}

/* ------------------------------------------------------------------------ */
/* a1': MLX affine quantize, 8 bits, group 64 (the north-star storage mode)  */
/*     call sites: Sources/KrillCore/CheckpointQuantizer.swift:255-260       */
/*     (casts to fp16 first so scales/biases are fp16),                      */
/*     Tests/KrillCoreTests/VerifyProfileTests.swift:70.                     */
/*     The algorithm itself lives in the third-party mlx library (not in     */
/*     the reference tree): restated from mlx's CPU affine quantize          */
/*     (mlx/backend/cpu/quantized.cpp, mlx 0.31 via mlx-swift 0.31.4).       */
/* ------------------------------------------------------------------------ */
/*
 * Per group of `group` fp16 values w (computed in binary32):
 *   s0   = max((w_max - w_min) / 255, 1e-7)
 *   side = |w_min| > |w_max|;  s = side ? s0 : -s0;  edge = side ? w_min : w_max
 *   q0   = rint(edge / s);  if q0 != 0: s = edge / q0, bias = edge  else bias = 0
 *   q    = min(rint((w - bias) / s), 255)      (always >= 0 by construction)
 *   scales, biases stored as fp16 (RNE).
 * Input in bf16 is first cast to fp16 (RNE), as the reference's affine path
 * casts to the storage dtype before quantizing.
 */
void oracle_quantize_mlx_affine(const uint16_t *x, int dt, int64_t n_rows, int D, int group,
                                uint8_t *q, uint16_t *scale_f16, uint16_t *bias_f16) {
    int G = D / group;
    float *w = (float *)malloc(sizeof(float) * (size_t)group);
    for (int64_t r = 0; r < n_rows; ++r) {
        for (int g = 0; g < G; ++g) {
            const uint16_t *xg = x + r * D + (int64_t)g * group;
            float wmin = INFINITY, wmax = -INFINITY;
            for (int i = 0; i < group; ++i) {
                float v = dt == DT_F16 ? oracle_f16_to_f32(xg[i])
                                       : oracle_f16_to_f32(oracle_f32_to_f16(oracle_bf16_to_f32(xg[i])));
                w[i] = v;
                if (v < wmin) wmin = v;
                if (v > wmax) wmax = v;
            }
            int side = fabsf(wmin) > fabsf(wmax);
            float s = (wmax - wmin) / 255.0f;
            if (!(s > 1e-7f)) s = 1e-7f;
            s = side ? s : -s;
            float edge = side ? wmin : wmax;
            float q0 = rintf(edge / s);
            float bias = 0.0f;
            if (q0 != 0.0f) {
                s = edge / q0;
                bias = edge;
            }
            for (int i = 0; i < group; ++i) {
                float n = rintf((w[i] - bias) / s);
                if (n > 255.0f) n = 255.0f;
                if (n < 0.0f) n = 0.0f; /* unreachable (see above); kept as a guard */
                q[r * D + (int64_t)g * group + i] = (uint8_t)n;
            }
            scale_f16[r * G + g] = oracle_f32_to_f16(s);
            bias_f16[r * G + g] = oracle_f32_to_f16(bias);
        }
    }
    free(w);
}

/* ------------------------------------------------------------------------ */
/* a3: QuantizedKVCache.dequantize  (QuantizedKVCache.swift:200-204)         */
/*     out = f16(f16(f16(q) * s) + z): two fp16 roundings, no fused FMA.     */
/* ------------------------------------------------------------------------ */
void oracle_dequant_ref_rows(const uint8_t *q, const uint16_t *s, const uint16_t *z,
                             int64_t n_rows, int D, uint16_t *out_f16) {
    for (int64_t r = 0; r < n_rows; ++r) {
        float sf = oracle_f16_to_f32(s[r]), zf = oracle_f16_to_f32(z[r]);
        for (int d = 0; d < D; ++d) {
            float prod = oracle_f16_to_f32(oracle_f32_to_f16((float)q[r * D + d] * sf));
            out_f16[r * D + d] = oracle_f32_to_f16(prod + zf);
        }
    }
}

/* Dequantize to binary64 values.  mode 0 (reference rows): the exact fp16
 * value the reference hands to attention.  mode 1 (affine groups): the exact
 * real value s*q + b of the stored fp16 scale/bias. */
void oracle_dequant_f64(const uint8_t *q, const uint16_t *s, const uint16_t *z,
                        int64_t n_rows, int D, int G, int mode, double *out) {
    for (int64_t r = 0; r < n_rows; ++r) {
        for (int d = 0; d < D; ++d) {
            int g = d / (D / G);
            float sf = oracle_f16_to_f32(s[r * G + g]), zf = oracle_f16_to_f32(z[r * G + g]);
            uint8_t qv = q[r * D + d];
            if (mode == 0) {
                float prod = oracle_f16_to_f32(oracle_f32_to_f16((float)qv * sf));
                out[r * D + d] = (double)oracle_f16_to_f32(oracle_f32_to_f16(prod + zf));
            } else {
                out[r * D + d] = (double)sf * (double)qv + (double)zf;
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* a7/a8: attention softmax(scale * q k^T + mask) v in binary64              */
/*   decode:  MLXFast.scaledDotProductAttention at                           */
/*            Sources/KrillCore/Attention.swift:95-98 (scale 1/sqrt(D), :44) */
/*            and Gemma4Model.swift:516-517 (scale 1.0);                     */
/*   masks:   BatchedDecode.swift:277-287 (left-pad), :299-312 (verify,      */
/*            block-causal), LlamaModel.swift:186-202 (cached causal).       */
/* A row r sees keys [0, limit[r]).  The -10000 additive mask of the          */
/* reference underflows the masked weights to exactly 0 (BatchedDecode.swift */
/* :22-28), so a length bound is the same function.                          */
/* ------------------------------------------------------------------------ */
void oracle_attention_f64(const double *q, const double *k, const double *v,
                          int NR, int T, int D, const int32_t *limit, double scale, double *out) {
    double *p = (double *)malloc(sizeof(double) * (size_t)(T > 0 ? T : 1));
    for (int r = 0; r < NR; ++r) {
        int lim = limit[r] < T ? limit[r] : T;
        double mx = -INFINITY;
        for (int t = 0; t < lim; ++t) {
            double acc = 0.0;
            for (int d = 0; d < D; ++d) acc += q[(int64_t)r * D + d] * k[(int64_t)t * D + d];
            p[t] = acc * scale;
            if (p[t] > mx) mx = p[t];
        }
        double l = 0.0;
        for (int t = 0; t < lim; ++t) {
            p[t] = exp(p[t] - mx);
            l += p[t];
        }
        for (int d = 0; d < D; ++d) {
            double acc = 0.0;
            for (int t = 0; t < lim; ++t) acc += p[t] * v[(int64_t)t * D + d];
            out[(int64_t)r * D + d] = lim > 0 ? acc / l : 0.0;
        }
    }
    free(p);
}

/* ------------------------------------------------------------------------ */
/* a5: stackCachesLeftPaddedQuantized (BatchedDecode.swift:96-151)           */
/* Rows r in [0,R), each [H, L_r, D] u8 + [H, L_r, G] f16 x2, are placed     */
/* right-aligned in [R, H, sMax, D] with u8 0 / f16 0 padding (:127-136).    */
/* Only the (q, scale, zero) triple of one of K or V is handled per call.    */
/* ------------------------------------------------------------------------ */
void oracle_stack_left_padded(const uint8_t *const *rows_q, const uint16_t *const *rows_s,
                              const uint16_t *const *rows_z, const int32_t *lens, int R, int H,
                              int D, int G, int sMax, uint8_t *out_q, uint16_t *out_s,
                              uint16_t *out_z) {
    memset(out_q, 0, (size_t)R * H * sMax * D);
    memset(out_s, 0, sizeof(uint16_t) * (size_t)R * H * sMax * G);
    memset(out_z, 0, sizeof(uint16_t) * (size_t)R * H * sMax * G);
    for (int r = 0; r < R; ++r) {
        int L = lens[r], pad = sMax - L;
        for (int h = 0; h < H; ++h) {
            memcpy(out_q + (((int64_t)r * H + h) * sMax + pad) * D, rows_q[r] + (int64_t)h * L * D,
                   (size_t)L * D);
            memcpy(out_s + (((int64_t)r * H + h) * sMax + pad) * G, rows_s[r] + (int64_t)h * L * G,
                   sizeof(uint16_t) * (size_t)L * G);
            memcpy(out_z + (((int64_t)r * H + h) * sMax + pad) * G, rows_z[r] + (int64_t)h * L * G,
                   sizeof(uint16_t) * (size_t)L * G);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* a10: prefix-cache key and longest common prefix                           */
/*   cacheKey: PrefixCache.swift:511-532 -- FNV-1a 64 over                   */
/*     schema(3) || dtype tag || utf8(modelId) || 0xFF || utf8(media) ||     */
/*     0xFF || tokens as 8-byte little-endian Int                            */
/*   commonPrefixLength: PrefixCache.swift:266-271                           */
/* ------------------------------------------------------------------------ */
uint64_t oracle_fnv1a64(const uint8_t *data, int64_t n, uint64_t h) {
    for (int64_t i = 0; i < n; ++i) {
        h ^= (uint64_t)data[i];
        h *= 1099511628211ull;
    }
    return h;
}

uint64_t oracle_prefix_key(const char *model_id, const char *media_hash, int dtype_tag,
                           const int64_t *tokens, int64_t n) {
    uint64_t h = 14695981039346656037ull;
    uint8_t hdr[2] = {3u, (uint8_t)dtype_tag};
    uint8_t ff = 0xFFu;
    h = oracle_fnv1a64(hdr, 2, h);
    h = oracle_fnv1a64((const uint8_t *)model_id, (int64_t)strlen(model_id), h);
    h = oracle_fnv1a64(&ff, 1, h);
    if (media_hash && media_hash[0]) h = oracle_fnv1a64((const uint8_t *)media_hash, (int64_t)strlen(media_hash), h);
    h = oracle_fnv1a64(&ff, 1, h);
    for (int64_t i = 0; i < n; ++i) {
        uint8_t b[8];
        uint64_t t = (uint64_t)tokens[i];
        for (int j = 0; j < 8; ++j) b[j] = (uint8_t)(t >> (8 * j));
        h = oracle_fnv1a64(b, 8, h);
    }
    return h;
}

int64_t oracle_common_prefix_length(const int64_t *a, int64_t na, const int64_t *b, int64_t nb) {
    int64_t n = na < nb ? na : nb, i = 0;
    while (i < n && a[i] == b[i]) ++i;
    return i;
}

/* ------------------------------------------------------------------------ */
/* CPU baseline: the reference's per-layer int8 decode step, timed beside    */
/* the GPU.  Per (sequence, layer) it does what QuantizedKVCache.update      */
/* (QuantizedKVCache.swift:49-75) followed by the SDPA call does:            */
/*   1. quantizePerHead the new K and V row (:51-52, :181-197)               */
/*   2. concatenated(...) the six tensors along the sequence axis -- a fresh */
/*      allocation and an O(T) copy per tensor (:55-61)                      */
/*   3. dequantize the WHOLE cache to fp16 (:72-73, :200-204)                */
/*   4. SDPA with GQA as MLX's composed ops run it (attention_mlx_composed  */
/*      in oracle.py): the query scaled in its own dtype (the scale a scalar */
/*      of that dtype), scores = q . K^T, a precise softmax, out = P . V,    */
/*      float32 accumulation; with fp16 queries the scores, the weights and  */
/*      the output are each rounded to fp16, with bf16 queries the products  */
/*      promote to float32 (bf16 x fp16) and stay there.                     */
/* Parallel over (sequence, kv-head) with OpenMP.                            */
/* ------------------------------------------------------------------------ */
typedef struct {
    uint8_t *qk, *qv;        /* [T*D] */
    uint16_t *ks, *kz, *vs, *vz; /* [T] */
    int T;
} base_row;

typedef struct {
    int layers, B, Hkv, Hq, D;
    base_row *rows; /* [layers][B][Hkv] */
    uint16_t *deq_k, *deq_v; /* per-thread scratch, sized lazily */
    int64_t scratch_T;
    int nthreads;
} base_session;

static uint64_t splitmix64(uint64_t *s) {
    uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

void *oracle_baseline_create(int layers, int B, int Hkv, int Hq, int D, const int32_t *lens,
                             uint64_t seed) {
    base_session *s = (base_session *)calloc(1, sizeof(base_session));
    s->layers = layers; s->B = B; s->Hkv = Hkv; s->Hq = Hq; s->D = D;
    s->rows = (base_row *)calloc((size_t)layers * B * Hkv, sizeof(base_row));
    uint64_t st = seed;
    for (int l = 0; l < layers; ++l)
        for (int b = 0; b < B; ++b)
            for (int h = 0; h < Hkv; ++h) {
                base_row *r = &s->rows[((int64_t)l * B + b) * Hkv + h];
                int T = lens[b];
                r->T = T;
                r->qk = (uint8_t *)malloc((size_t)T * D + 1);
                r->qv = (uint8_t *)malloc((size_t)T * D + 1);
                r->ks = (uint16_t *)malloc(2 * (size_t)T + 2);
                r->kz = (uint16_t *)malloc(2 * (size_t)T + 2);
                r->vs = (uint16_t *)malloc(2 * (size_t)T + 2);
                r->vz = (uint16_t *)malloc(2 * (size_t)T + 2);
                for (int64_t i = 0; i < (int64_t)T * D; i += 8) {
                    uint64_t w = splitmix64(&st);
                    for (int j = 0; j < 8 && i + j < (int64_t)T * D; ++j) {
                        r->qk[i + j] = (uint8_t)(w >> (8 * j));
                        r->qv[i + j] = (uint8_t)(w >> (8 * j + 4));
                    }
                }
                for (int t = 0; t < T; ++t) {
                    r->ks[t] = r->vs[t] = oracle_f32_to_f16(6.0f / 255.0f);
                    r->kz[t] = r->vz[t] = oracle_f32_to_f16(-3.0f);
                }
            }
#ifdef _OPENMP
    s->nthreads = omp_get_max_threads();
#else
    s->nthreads = 1;
#endif
    return s;
}

void oracle_baseline_destroy(void *h) {
    base_session *s = (base_session *)h;
    if (!s) return;
    for (int64_t i = 0; i < (int64_t)s->layers * s->B * s->Hkv; ++i) {
        base_row *r = &s->rows[i];
        free(r->qk); free(r->qv); free(r->ks); free(r->kz); free(r->vs); free(r->vz);
    }
    free(s->rows);
    free(s);
}

static void *grow_copy(void *old, size_t old_bytes, size_t new_bytes) {
    /* concatenated([existing, new]) allocates a new array and copies */
    void *n = malloc(new_bytes);
    memcpy(n, old, old_bytes);
    free(old);
    return n;
}

int oracle_baseline_threads(void *h) { return ((base_session *)h)->nthreads; }

/* Threads of the following steps (1 = the single-thread figure). */
void oracle_baseline_set_threads(void *h, int n) {
#ifdef _OPENMP
    ((base_session *)h)->nthreads = n > 0 ? n : 1;
#else
    (void)n;
    ((base_session *)h)->nthreads = 1;
#endif
}

/* One decode step over all layers.  k_new/v_new: [layers][B][Hkv][D] bf16
 * (or f16 by dt), q: [layers][B][Hq][D] in dt, out: [layers][B][Hq][D] f32. */
void oracle_baseline_step(void *h, const uint16_t *q, const uint16_t *k_new, const uint16_t *v_new,
                          int dt, float scale, float *out, int layers_to_run) {
    base_session *s = (base_session *)h;
    int B = s->B, Hkv = s->Hkv, Hq = s->Hq, D = s->D, R = Hq / Hkv;
    if (layers_to_run <= 0 || layers_to_run > s->layers) layers_to_run = s->layers;
    for (int l = 0; l < layers_to_run; ++l) {
#pragma omp parallel for schedule(dynamic, 1) num_threads(s->nthreads)
        for (int bh = 0; bh < B * Hkv; ++bh) {
            int b = bh / Hkv, hk = bh % Hkv;
            base_row *r = &s->rows[((int64_t)l * B + b) * Hkv + hk];
            const uint16_t *kn = k_new + (((int64_t)l * B + b) * Hkv + hk) * D;
            const uint16_t *vn = v_new + (((int64_t)l * B + b) * Hkv + hk) * D;
            uint8_t qk1[512], qv1[512];
            uint16_t ks1, kz1, vs1, vz1;
            oracle_quantize_ref_rows(kn, dt, 1, D, qk1, &ks1, &kz1);
            oracle_quantize_ref_rows(vn, dt, 1, D, qv1, &vs1, &vz1);
            int T = r->T;
            r->qk = (uint8_t *)grow_copy(r->qk, (size_t)T * D, (size_t)(T + 1) * D);
            r->qv = (uint8_t *)grow_copy(r->qv, (size_t)T * D, (size_t)(T + 1) * D);
            r->ks = (uint16_t *)grow_copy(r->ks, 2 * (size_t)T, 2 * (size_t)(T + 1));
            r->kz = (uint16_t *)grow_copy(r->kz, 2 * (size_t)T, 2 * (size_t)(T + 1));
            r->vs = (uint16_t *)grow_copy(r->vs, 2 * (size_t)T, 2 * (size_t)(T + 1));
            r->vz = (uint16_t *)grow_copy(r->vz, 2 * (size_t)T, 2 * (size_t)(T + 1));
            memcpy(r->qk + (int64_t)T * D, qk1, D);
            memcpy(r->qv + (int64_t)T * D, qv1, D);
            r->ks[T] = ks1; r->kz[T] = kz1; r->vs[T] = vs1; r->vz[T] = vz1;
            T += 1;
            r->T = T;
            /* full-cache dequant to fp16 (transient, as in update()) */
            uint16_t *dk = (uint16_t *)malloc(2 * (size_t)T * D);
            uint16_t *dv = (uint16_t *)malloc(2 * (size_t)T * D);
            oracle_dequant_ref_rows(r->qk, r->ks, r->kz, T, D, dk);
            oracle_dequant_ref_rows(r->qv, r->vs, r->vz, T, D, dv);
            float *sc = (float *)malloc(sizeof(float) * (size_t)T);
            float *kf = (float *)malloc(sizeof(float) * (size_t)T * D);
            float *vf = (float *)malloc(sizeof(float) * (size_t)T * D);
            for (int64_t i = 0; i < (int64_t)T * D; ++i) {
                kf[i] = oracle_f16_to_f32(dk[i]);
                vf[i] = oracle_f16_to_f32(dv[i]);
            }
            const int half = dt == DT_F16;  /* fp16 queries: fp16 products */
            const float sdt = dt_round(scale, dt);
            for (int j = 0; j < R; ++j) {
                int hq = hk * R + j;
                const uint16_t *qr = q + (((int64_t)l * B + b) * Hq + hq) * D;
                float qf[512];
                for (int d = 0; d < D; ++d) qf[d] = dt_round(dt_to_f32(qr[d], dt) * sdt, dt);
                float mx = -INFINITY;
                for (int t = 0; t < T; ++t) {
                    float acc = 0.0f;
                    const float *kr = kf + (int64_t)t * D;
                    for (int d = 0; d < D; ++d) acc += qf[d] * kr[d];
                    sc[t] = half ? dt_round(acc, DT_F16) : acc;
                    if (sc[t] > mx) mx = sc[t];
                }
                float lsum = 0.0f;
                for (int t = 0; t < T; ++t) { sc[t] = expf(sc[t] - mx); lsum += sc[t]; }
                float *o = out + (((int64_t)l * B + b) * Hq + hq) * D;
                for (int d = 0; d < D; ++d) o[d] = 0.0f;
                for (int t = 0; t < T; ++t) {
                    float p = sc[t] / lsum;
                    if (half) p = dt_round(p, DT_F16);
                    const float *vr = vf + (int64_t)t * D;
                    for (int d = 0; d < D; ++d) o[d] += p * vr[d];
                }
                if (half)
                    for (int d = 0; d < D; ++d) o[d] = dt_round(o[d], DT_F16);
            }
            free(dk); free(dv); free(sc); free(kf); free(vf);
        }
    }
}

/* Array forms of the conversions (for the exhaustive conversion tests). */
void oracle_f16_to_f32_array(const uint16_t *h, int64_t n, float *out) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_f16_to_f32(h[i]);
}
void oracle_f32_to_f16_array(const float *f, int64_t n, uint16_t *out) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_f16(f[i]);
}
void oracle_f32_to_bf16_array(const float *f, int64_t n, uint16_t *out) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_bf16(f[i]);
}
