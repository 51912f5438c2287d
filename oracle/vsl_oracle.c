/*
 * vsl_oracle.c -- CPU restatement of Vulkan-Symbiote-Loader's per-token forward pass.
 *
 * TEST INFRASTRUCTURE ONLY (the oracle).  Loaded by tests/, the smoke() entry point and the
 * cpu_baseline leg of bench.py; never by the product.
 *
 * Parity pins (what checks each function; see tests/test_oracle.py):
 *   orc_h2f / orc_f2h        exhaustive over all 65,536 binary16 patterns vs numpy float16,
 *                            and every float16 round trip; RNE ties checked at half-ulp points
 *   orc_fnv1a64              published FNV-1a-64 test vectors ("" and "a", "foobar")
 *   orc_philox4x32_10        Random123 known-answer vectors (Salmon et al., SC'11)
 *   GGUF parse               hand-computed byte offsets of a file assembled byte by byte in the
 *                            test, both tensor-type conventions, the reference's error codes
 *   orc_rmsnorm              closed form: output RMS == 1 for unit gains, scale invariance
 *   orc_rope                 pos 0 identity, norm preservation, <R_m q, R_n k> depends on m-n only,
 *                            and the adjacent-pair convention against a hand-rotated vector
 *   orc_attention_decode     one-key attention == V, uniform scores == mean of V, brute force fp64
 *   windowed attention       uniform scores over one-hot values give 1/|A| exactly on the attended
 *                            set A, written out literally per (len, window, globals, threshold);
 *                            keys outside A perturbed without effect; threshold not reached == dense
 *   orc_gemm_nt              fp64 numpy matmul on the GEMV-sweep shapes (reduced N)
 *   orc_swiglu               closed forms silu(0)=0, silu(x)->x
 *   orc_forward / generate   tiny-config logits vs an independent transformers LlamaForCausalLM
 *                            built from a local config with the RoPE pair permutation applied to
 *                            Wq/Wk; committed golden token ids and logits
 *   orc_sample               greedy = lowest index of the max; seeded top-k vs a numpy restatement
 *                            of Utils.cpp:140-172 driven by the Philox stream
 *   orc_dequant              hand-assembled Q4_0 / Q4_1 / Q8_0 blocks with literal expected values
 *                            (nibble order of each convention, every int8 code, the scale helper's
 *                            unsigned subnormals, partial and truncated final blocks, -20 for
 *                            other quantized ids) and a bound |x - dq(q(x))| <= d/2 against an
 *                            independent numpy quantizer
 */
#define _GNU_SOURCE
#include "vsl_oracle.h"

#include <errno.h>
#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#if defined(__x86_64__)
#include <immintrin.h>
#endif

/* =========================================================================================
 * scalar helpers
 * ========================================================================================= */

/* IEEE-754 binary16 -> binary32.  Same cases as GGUFLoader.cpp:1225-1262 (zero, subnormal,
 * inf/NaN, normal); the reference maps every NaN to +qNaN, here the sign and payload are kept
 * (NaN weights do not occur in the synthetic models, so the difference is never observed). */
float orc_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1F;
    uint32_t man = h & 0x3FF;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: value = man * 2^-24 */
            float v = (float)man * 5.9604644775390625e-08f;
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* binary32 -> binary16 with round-to-nearest-even; overflow -> inf, NaN stays NaN. */
uint16_t orc_f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7FFFFFFFu;
    if (absx >= 0x7F800000u) { /* inf or NaN */
        uint32_t man = absx & 0x7FFFFFu;
        return (uint16_t)(sign | 0x7C00u | (man ? (0x200u | (man >> 13)) : 0));
    }
    if (absx >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to inf */
    if (absx < 0x38800000u) {                                    /* below 2^-14: subnormal/zero */
        if (absx < 0x33000000u) return (uint16_t)sign;           /* < 2^-25 rounds to 0 */
        uint32_t e = absx >> 23;
        uint32_t m = (absx & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126 - e; /* 14..24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (absx >> 23) - 112;
    uint32_t m = absx & 0x7FFFFFu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++;
    return (uint16_t)(sign | q);
}

static float g_h2f_table[65536];
static int g_h2f_ready = 0;
static void h2f_table_init(void) {
    if (g_h2f_ready) return;
    for (uint32_t i = 0; i < 65536; ++i) g_h2f_table[i] = orc_h2f((uint16_t)i);
    g_h2f_ready = 1;
}

/* FNV-1a recurrence with an explicit offset basis. */
uint64_t orc_fnv1a64_basis(const char* s, uint64_t basis) {
    uint64_t h = basis;
    for (const unsigned char* p = (const unsigned char*)s; *p; ++p) {
        h ^= *p;
        h *= 1099511628211ULL;
    }
    return h;
}

/* hash_string, Utils.cpp:9-16.  The reference's offset basis is 1469598103934665603, one digit
 * short of FNV's published 14695981039346656037; it is kept as written. */
uint64_t orc_fnv1a64(const char* s) { return orc_fnv1a64_basis(s, 1469598103934665603ULL); }

/* Philox4x32-10, J. Salmon et al., "Parallel Random Numbers: As Easy as 1, 2, 3", SC'11. */
void orc_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
    uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
    uint32_t k0 = key_in[0], k1 = key_in[1];
    for (int r = 0; r < 10; ++r) {
        uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
        uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        uint32_t n0 = hi1 ^ c1 ^ k0;
        uint32_t n2 = hi0 ^ c3 ^ k1;
        c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

static void derive_key(uint64_t seed, const char* name, uint32_t key[2]) {
    uint64_t k = orc_fnv1a64(name) ^ (seed * 0x9E3779B97F4A7C15ULL);
    key[0] = (uint32_t)k;
    key[1] = (uint32_t)(k >> 32);
}

static int g_threads = 0;
int orc_num_threads(void) {
#ifdef _OPENMP
    return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
    return 1;
#endif
}
void orc_set_num_threads(int n) {
    g_threads = n;
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#endif
}

/* =========================================================================================
 * synthetic data generator (shared specification with the product's generators)
 * ========================================================================================= */
static inline void box_muller(uint32_t a, uint32_t b, double* z0, double* z1) {
    double u1 = ((double)a + 1.0) * (1.0 / 4294967296.0); /* (0, 1] */
    double u2 = (double)b * (1.0 / 4294967296.0);         /* [0, 1) */
    double r = sqrt(-2.0 * log(u1));
    double t = 6.283185307179586476925286766559 * u2;
    *z0 = r * cos(t);
    *z1 = r * sin(t);
}

void orc_fill_normal(void* out, int out_dtype, uint64_t n, uint64_t seed, const char* name,
                     float mean, float stddev) {
    uint32_t key[2];
    derive_key(seed, name, key);
    uint64_t nblk = (n + 3) / 4;
#pragma omp parallel for schedule(static)
    for (uint64_t b = 0; b < nblk; ++b) {
        uint32_t ctr[4] = {(uint32_t)b, (uint32_t)(b >> 32), 0, 0}, r[4];
        orc_philox4x32_10(ctr, key, r);
        double z[4];
        box_muller(r[0], r[1], &z[0], &z[1]);
        box_muller(r[2], r[3], &z[2], &z[3]);
        for (int j = 0; j < 4; ++j) {
            uint64_t e = b * 4 + j;
            if (e >= n) break;
            float v = (float)((double)mean + (double)stddev * z[j]);
            if (out_dtype == ORC_F16)
                ((uint16_t*)out)[e] = orc_f2h(v);
            else
                ((float*)out)[e] = v;
        }
    }
}

void orc_random_ids(uint32_t* out, uint32_t n, uint32_t vocab, uint64_t seed, const char* name) {
    uint32_t key[2];
    derive_key(seed, name, key);
    for (uint32_t i = 0; i < n; i += 4) {
        uint32_t ctr[4] = {i / 4, 0, 0, 0}, r[4];
        orc_philox4x32_10(ctr, key, r);
        for (uint32_t j = 0; j < 4 && i + j < n; ++j)
            out[i + j] = (uint32_t)(((uint64_t)r[j] * vocab) >> 32);
    }
}

/* =========================================================================================
 * GGUF (GGUFLoader.cpp:625-980, 1085-1119)
 * ========================================================================================= */
/* metadata value types: GGUFLoader.h:18-31 (identical to ggml's metadata ids) */
enum { MV_U8 = 0, MV_I8, MV_U16, MV_I16, MV_U32, MV_I32, MV_F32, MV_BOOL, MV_STR, MV_ARR, MV_U64, MV_I64, MV_F64 };

typedef struct {
    char* key;
    uint32_t type;
    const uint8_t* val; /* points into the mapping: scalar bytes, or (len u64 + bytes) for strings */
    uint64_t val_len;
} gkv;

typedef struct {
    char* name;
    uint32_t n_dims;
    uint64_t dims[4];
    uint32_t raw_type;
    uint64_t offset, data_offset, data_size, n_elem;
    int kind;  /* 0 f32, 1 f16, -1 unsupported */
    int quant; /* 1 for a block-quantized type that orc_dequant expands to fp32 */
} gti;

struct orc_gguf {
    int fd;
    const uint8_t* map;
    size_t size;
    uint32_t version;
    uint64_t n_tensors, n_kv;
    gkv* kvs;
    gti* tis;
    uint64_t data_start;
    int convention; /* 0 reference ids (F32=6, F16=48), 1 ggml ids (F32=0, F16=1) */
};

typedef struct { const uint8_t* p; const uint8_t* end; } cursor;

static int cur_take(cursor* c, void* dst, size_t n) {
    if ((size_t)(c->end - c->p) < n) return -1;
    if (dst) memcpy(dst, c->p, n);
    c->p += n;
    return 0;
}

/* read_value (GGUFLoader.cpp:913-980): skip one value of type t, return 0 on success */
static int skip_value(cursor* c, uint32_t t, int depth) {
    if (depth > 4) return -1;
    switch (t) {
        case MV_U8: case MV_I8: case MV_BOOL: return cur_take(c, NULL, 1);
        case MV_U16: case MV_I16: return cur_take(c, NULL, 2);
        case MV_U32: case MV_I32: case MV_F32: return cur_take(c, NULL, 4);
        case MV_U64: case MV_I64: case MV_F64: return cur_take(c, NULL, 8);
        case MV_STR: {
            uint64_t len;
            if (cur_take(c, &len, 8)) return -1;
            return cur_take(c, NULL, len);
        }
        case MV_ARR: {
            uint32_t et;
            uint64_t cnt;
            if (cur_take(c, &et, 4) || cur_take(c, &cnt, 8)) return -1;
            for (uint64_t i = 0; i < cnt; ++i)
                if (skip_value(c, et, depth + 1)) return -1;
            return 0;
        }
        default: return -1; /* the reference returns false for any other type */
    }
}

static uint64_t ref_type_size(uint32_t t, uint64_t n) { /* calculate_tensor_data_size :1085-1119 */
    switch (t) {
        case 0: case 1: return n;
        case 2: case 3: case 48: case 47: return n * 2;
        case 4: case 5: case 6: return n * 4;
        case 10: case 11: case 12: return n * 8;
        case 13: return (n / 32) * 18 + ((n % 32) ? 18 : 0);
        case 14: return (n / 32) * 20 + ((n % 32) ? 20 : 0);
        case 15: return (n / 32) * 22 + ((n % 32) ? 22 : 0);
        case 16: return (n / 32) * 24 + ((n % 32) ? 24 : 0);
        case 17: return (n / 32) * 34 + ((n % 32) ? 34 : 0);
        default: return n * 4;
    }
}

static uint64_t ggml_type_size(uint32_t t, uint64_t n) {
    switch (t) {
        case 0: return n * 4;                /* F32 */
        case 1: return n * 2;                /* F16 */
        case 2: return (n / 32) * 18;        /* Q4_0 */
        case 3: return (n / 32) * 20;        /* Q4_1 */
        case 8: return (n / 32) * 34;        /* Q8_0 */
        case 30: return n * 2;               /* BF16 */
        default: return 0;
    }
}

/* Block formats expanded by orc_dequant: 0 Q4_0, 1 Q4_1, 2 Q8_0, -1 anything else.  Reference
 * ids Q4_0 = 13, Q4_1 = 14, Q8_0 = 17 (GGUFLoader.h:18-73); ggml ids 2, 3, 8 (ggml's published
 * type enum, which the reference does not use). */
static int quant_format(uint32_t raw_type, int convention) {
    if (convention == 0) return raw_type == 13 ? 0 : raw_type == 14 ? 1 : raw_type == 17 ? 2 : -1;
    return raw_type == 2 ? 0 : raw_type == 3 ? 1 : raw_type == 8 ? 2 : -1;
}

/* The scale conversion local to dequantize_tensor (GGUFLoader.cpp:1132-1149).  It differs from
 * IEEE binary16 only where the exponent field is 0: a subnormal becomes mantissa * 2^-24 with
 * its sign dropped, and -0 becomes +0.  Infinities and NaNs keep their sign. */
static float ref_block_scale(uint16_t h) {
    const uint32_t exp = (h >> 10) & 0x1F, man = h & 0x3FF;
    if (exp == 0) return man == 0 ? 0.0f : (float)man * 5.9604644775390625e-08f; /* exact */
    return orc_h2f(h);
}

/* dequantize_tensor (GGUFLoader.cpp:1121-1223) for reference-convention files; for ggml-id files
 * the same three formats with ggml's published block layout.
 *   Q4_0  fp16 d, 16 bytes   x = (nibble - 8) * d
 *   Q4_1  fp16 d, fp16 m, 16 bytes   x = nibble * d + m
 *   Q8_0  fp16 d, 32 int8    x = q * d
 * Nibble order: the reference reads byte i as elements 2i (low nibble) and 2i+1 (high nibble)
 * (:1163-1168, :1187-1192); ggml stores element j < 16 in the low nibble of byte j and element
 * j + 16 in its high nibble.  Scales: the reference's helper above, ggml's exact binary16.
 * Every product q * d is exact in binary32 (at most 8 + 11 significant bits), so the result does
 * not depend on evaluation order or FMA contraction.
 * Blocks are read while a whole block remains in `size` bytes (the loop guard at :1157, :1178,
 * :1203); the last block may be partial (n not a multiple of 32).  Returns the number of floats
 * written, which is below n when the data runs out, or -20 for any other type. */
int64_t orc_dequant(const void* data, uint64_t size, uint32_t raw_type, int convention, uint64_t n, float* out) {
    const int q = quant_format(raw_type, convention);
    if (q < 0) return -20;
    const uint8_t* p = (const uint8_t*)data;
    const uint64_t bb = q == 0 ? 18 : (q == 1 ? 20 : 34);
    const uint64_t nb = (n + 31) / 32;
    uint64_t w = 0;
    for (uint64_t b = 0; b < nb && (b + 1) * bb <= size; ++b) {
        const uint8_t* blk = p + b * bb;
        uint16_t hd, hm = 0;
        memcpy(&hd, blk, 2);
        if (q == 1) memcpy(&hm, blk + 2, 2);
        const float d = convention == 0 ? ref_block_scale(hd) : orc_h2f(hd);
        const float m = q != 1 ? 0.0f : (convention == 0 ? ref_block_scale(hm) : orc_h2f(hm));
        const uint8_t* qs = blk + (q == 1 ? 4 : 2);
        for (int j = 0; j < 32 && w < n; ++j) {
            float v;
            if (q == 2) {
                v = (float)(int8_t)qs[j] * d;
            } else {
                const int nib = convention == 0 ? ((j & 1) ? qs[j >> 1] >> 4 : qs[j >> 1] & 15)
                                                : (j < 16 ? qs[j] & 15 : qs[j - 16] >> 4);
                v = q == 0 ? (float)(nib - 8) * d : (float)nib * d + m;
            }
            out[w++] = v;
        }
    }
    return (int64_t)w;
}

static const gkv* find_kv(const orc_gguf* g, const char* key) {
    for (uint64_t i = 0; i < g->n_kv; ++i)
        if (strcmp(g->kvs[i].key, key) == 0) return &g->kvs[i];
    return NULL;
}

void orc_gguf_close(orc_gguf* g) {
    if (!g) return;
    if (g->kvs) {
        for (uint64_t i = 0; i < g->n_kv; ++i) free(g->kvs[i].key);
        free(g->kvs);
    }
    if (g->tis) {
        for (uint64_t i = 0; i < g->n_tensors; ++i) free(g->tis[i].name);
        free(g->tis);
    }
    if (g->map && g->map != MAP_FAILED) munmap((void*)g->map, g->size);
    if (g->fd >= 0) close(g->fd);
    free(g);
}

int orc_gguf_open(const char* path, orc_gguf** out) {
    *out = NULL;
    orc_gguf* g = (orc_gguf*)calloc(1, sizeof(orc_gguf));
    g->fd = open(path, O_RDONLY);
    if (g->fd < 0) { free(g); return -1; }
    struct stat st;
    if (fstat(g->fd, &st) != 0) { orc_gguf_close(g); return -1; }
    g->size = (size_t)st.st_size;
    if (g->size < 24) { orc_gguf_close(g); return -2; }
    g->map = (const uint8_t*)mmap(NULL, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (g->map == MAP_FAILED) { g->map = NULL; orc_gguf_close(g); return -1; }
    cursor c = {g->map, g->map + g->size};
    uint32_t magic = 0;
    cur_take(&c, &magic, 4);
    if (magic != 0x46554747u) { orc_gguf_close(g); return -2; }
    cur_take(&c, &g->version, 4);
    cur_take(&c, &g->n_tensors, 8);
    cur_take(&c, &g->n_kv, 8);
    if (g->n_kv > (g->size / 12) || g->n_tensors > (g->size / 24)) { orc_gguf_close(g); return -3; }
    g->kvs = (gkv*)calloc(g->n_kv ? g->n_kv : 1, sizeof(gkv));
    for (uint64_t i = 0; i < g->n_kv; ++i) { /* parse_metadata :847-874 */
        uint64_t klen;
        if (cur_take(&c, &klen, 8) || klen > (uint64_t)(c.end - c.p)) { orc_gguf_close(g); return -3; }
        g->kvs[i].key = strndup((const char*)c.p, klen);
        c.p += klen;
        if (cur_take(&c, &g->kvs[i].type, 4)) { orc_gguf_close(g); return -3; }
        const uint8_t* vstart = c.p;
        if (skip_value(&c, g->kvs[i].type, 0)) { orc_gguf_close(g); return -3; }
        g->kvs[i].val = vstart;
        g->kvs[i].val_len = (uint64_t)(c.p - vstart);
    }
    g->tis = (gti*)calloc(g->n_tensors ? g->n_tensors : 1, sizeof(gti));
    for (uint64_t i = 0; i < g->n_tensors; ++i) { /* parse_tensor_info :876-911 */
        gti* t = &g->tis[i];
        uint64_t nlen;
        if (cur_take(&c, &nlen, 8) || nlen > (uint64_t)(c.end - c.p)) { orc_gguf_close(g); return -4; }
        t->name = strndup((const char*)c.p, nlen);
        c.p += nlen;
        if (cur_take(&c, &t->n_dims, 4) || t->n_dims > 4) { orc_gguf_close(g); return -4; }
        t->n_elem = 1;
        for (uint32_t d = 0; d < t->n_dims; ++d) {
            if (cur_take(&c, &t->dims[d], 8)) { orc_gguf_close(g); return -4; }
            t->n_elem *= t->dims[d];
        }
        if (cur_take(&c, &t->raw_type, 4) || cur_take(&c, &t->offset, 8)) { orc_gguf_close(g); return -4; }
    }
    uint64_t after_infos = (uint64_t)(c.p - g->map);

    /* tensor-type convention: explicit key, else inferred from the ids present */
    g->convention = 0;
    const gkv* conv = find_kv(g, "vsl.tensor_type_convention");
    if (conv && conv->type == MV_STR) {
        uint64_t l;
        memcpy(&l, conv->val, 8);
        g->convention = (l == 4 && memcmp(conv->val + 8, "ggml", 4) == 0) ? 1 : 0;
    } else if (find_kv(g, "general.alignment")) {
        g->convention = 1;
    } else {
        int has_ggml = 0, has_ref = 0;
        for (uint64_t i = 0; i < g->n_tensors; ++i) {
            uint32_t t = g->tis[i].raw_type;
            if (t == 0 || t == 1 || t == 2 || t == 3 || t == 8) has_ggml = 1;
            if (t == 48) has_ref = 1;
        }
        g->convention = (has_ggml && !has_ref) ? 1 : 0;
    }
    if (g->convention == 0) {
        g->data_start = after_infos; /* reference: tellg() right after the infos (:653) */
    } else {
        uint32_t align = 32;
        const gkv* a = find_kv(g, "general.alignment");
        if (a && a->type == MV_U32) memcpy(&align, a->val, 4);
        if (align == 0) align = 32;
        g->data_start = (after_infos + align - 1) / align * align;
    }
    for (uint64_t i = 0; i < g->n_tensors; ++i) {
        gti* t = &g->tis[i];
        t->data_offset = g->data_start + t->offset;
        if (g->convention == 0) {
            t->data_size = ref_type_size(t->raw_type, t->n_elem);
            t->kind = t->raw_type == 6 ? ORC_F32 : (t->raw_type == 48 ? ORC_F16 : -1);
            t->quant = quant_format(t->raw_type, 0) >= 0;
        } else {
            t->data_size = ggml_type_size(t->raw_type, t->n_elem);
            t->kind = t->raw_type == 0 ? ORC_F32 : (t->raw_type == 1 ? ORC_F16 : -1);
            /* ggml blocks never straddle rows: ne0 must be a whole number of blocks */
            t->quant = quant_format(t->raw_type, 1) >= 0 && t->n_dims > 0 && t->dims[0] % 32 == 0;
        }
    }
    *out = g;
    return 0;
}

uint64_t orc_gguf_tensor_count(const orc_gguf* g) { return g->n_tensors; }
uint64_t orc_gguf_metadata_count(const orc_gguf* g) { return g->n_kv; }
uint32_t orc_gguf_version(const orc_gguf* g) { return g->version; }
uint64_t orc_gguf_data_start(const orc_gguf* g) { return g->data_start; }
int orc_gguf_convention(const orc_gguf* g) { return g->convention; }

int orc_gguf_find(const orc_gguf* g, const char* name) {
    for (uint64_t i = 0; i < g->n_tensors; ++i)
        if (strcmp(g->tis[i].name, name) == 0) return (int)i;
    return -1;
}

int orc_gguf_tensor_info(const orc_gguf* g, int idx, char* name_out, size_t name_cap,
                         uint32_t* n_dims, uint64_t dims[4], uint32_t* raw_type,
                         uint64_t* data_offset, uint64_t* data_size) {
    if (idx < 0 || (uint64_t)idx >= g->n_tensors) return -30;
    const gti* t = &g->tis[idx];
    if (name_out && name_cap) {
        strncpy(name_out, t->name, name_cap - 1);
        name_out[name_cap - 1] = 0;
    }
    if (n_dims) *n_dims = t->n_dims;
    if (dims) for (int d = 0; d < 4; ++d) dims[d] = d < (int)t->n_dims ? t->dims[d] : 1;
    if (raw_type) *raw_type = t->raw_type;
    if (data_offset) *data_offset = t->data_offset;
    if (data_size) *data_size = t->data_size;
    return 0;
}

static const void* tensor_ptr(const orc_gguf* g, const gti* t) {
    if (t->data_offset + t->data_size > g->size) return NULL;
    return g->map + t->data_offset;
}

int64_t orc_gguf_read_f32(const orc_gguf* g, const char* name, float* out, uint64_t cap) {
    int i = orc_gguf_find(g, name);
    if (i < 0) return -30;
    const gti* t = &g->tis[i];
    const void* p = tensor_ptr(g, t);
    if (!p) return -11;
    if (t->quant) {
        if (t->n_elem > cap) return -11;
        return orc_dequant(p, t->data_size, t->raw_type, g->convention, t->n_elem, out);
    }
    if (quant_format(t->raw_type, g->convention) >= 0 ||
        (g->convention == 0 ? (t->raw_type >= 13 && t->raw_type <= 53 && t->raw_type != 48)
                            : (t->raw_type >= 2 && t->raw_type != 30)))
        return -20; /* other quantized ids reach dequantize_tensor's default case (:1219-1220) */
    if (t->kind < 0) return -12;
    if (t->n_elem > cap) return -11;
    if (t->kind == ORC_F32) {
        memcpy(out, p, t->n_elem * 4);
    } else {
        const uint16_t* h = (const uint16_t*)p;
        for (uint64_t e = 0; e < t->n_elem; ++e) out[e] = orc_h2f(h[e]);
    }
    return (int64_t)t->n_elem;
}

int orc_gguf_get_u32(const orc_gguf* g, const char* key, uint32_t* v) {
    const gkv* kv = find_kv(g, key);
    if (!kv || kv->type != MV_U32) return -1; /* get_uint32 requires the exact type (:39-42) */
    memcpy(v, kv->val, 4);
    return 0;
}

int orc_gguf_get_f32(const orc_gguf* g, const char* key, float* v) {
    const gkv* kv = find_kv(g, key);
    if (!kv || kv->type != MV_F32) return -1;
    memcpy(v, kv->val, 4);
    return 0;
}

int orc_gguf_get_str(const orc_gguf* g, const char* key, char* out, size_t cap) {
    const gkv* kv = find_kv(g, key);
    if (!kv || kv->type != MV_STR || cap == 0) return -1;
    uint64_t l;
    memcpy(&l, kv->val, 8);
    size_t n = l < cap - 1 ? (size_t)l : cap - 1;
    memcpy(out, kv->val + 8, n);
    out[n] = 0;
    return 0;
}

void orc_gguf_model_config(const orc_gguf* g, orc_config* cfg) {
    /* defaults: ModelConfig, Common.h:56-76 */
    cfg->hidden_size = 4096; cfg->num_layers = 32; cfg->num_heads = 32; cfg->num_kv_heads = 32;
    cfg->intermediate_size = 11008; cfg->vocab_size = 32000; cfg->rope_theta = 10000.0f;
    cfg->max_position_embeddings = 2048; cfg->rms_eps = 1e-5f;
    uint32_t v;
    float f;
    /* a key that is present with another type reads as 0 (get_uint32 :39-42) */
    const gkv* kv;
    if ((kv = find_kv(g, "llama.embedding_length"))) cfg->hidden_size = orc_gguf_get_u32(g, "llama.embedding_length", &v) ? 0 : v;
    else if ((kv = find_kv(g, "general.embedding_length"))) cfg->hidden_size = orc_gguf_get_u32(g, "general.embedding_length", &v) ? 0 : v;
    if ((kv = find_kv(g, "llama.block_count"))) cfg->num_layers = orc_gguf_get_u32(g, "llama.block_count", &v) ? 0 : v;
    else if ((kv = find_kv(g, "general.block_count"))) cfg->num_layers = orc_gguf_get_u32(g, "general.block_count", &v) ? 0 : v;
    if ((kv = find_kv(g, "llama.attention.head_count"))) cfg->num_heads = orc_gguf_get_u32(g, "llama.attention.head_count", &v) ? 0 : v;
    if ((kv = find_kv(g, "llama.attention.head_count_kv"))) cfg->num_kv_heads = orc_gguf_get_u32(g, "llama.attention.head_count_kv", &v) ? 0 : v;
    else cfg->num_kv_heads = cfg->num_heads;
    if ((kv = find_kv(g, "llama.feed_forward_length"))) cfg->intermediate_size = orc_gguf_get_u32(g, "llama.feed_forward_length", &v) ? 0 : v;
    if ((kv = find_kv(g, "llama.vocab_size"))) cfg->vocab_size = orc_gguf_get_u32(g, "llama.vocab_size", &v) ? 0 : v;
    if ((kv = find_kv(g, "llama.rope.freq_base"))) cfg->rope_theta = orc_gguf_get_f32(g, "llama.rope.freq_base", &f) ? 0.0f : f;
    if ((kv = find_kv(g, "llama.context_length"))) cfg->max_position_embeddings = orc_gguf_get_u32(g, "llama.context_length", &v) ? 0 : v;
    if (!orc_gguf_get_f32(g, "llama.attention.layer_norm_rms_epsilon", &f)) cfg->rms_eps = f;
    cfg->head_dim = cfg->num_heads ? cfg->hidden_size / cfg->num_heads : 0;
    (void)kv;
}

/* =========================================================================================
 * model
 * ========================================================================================= */
typedef struct { const void* p; int t; } wref;

typedef struct {
    float* attn_norm;
    float* ffn_norm;
    wref q, k, v, o, gate, up, down;
} orc_layer;

struct orc_model {
    orc_config cfg;
    uint32_t win, n_global, win_threshold; /* windowed attention; win_threshold UINT32_MAX = dense */
    wref tok_embd, output;
    float* out_norm;
    orc_layer* layers;
    void** owned;
    size_t n_owned, cap_owned;
    orc_gguf* gguf;
};

static void own(orc_model* m, void* p) {
    if (m->n_owned == m->cap_owned) {
        m->cap_owned = m->cap_owned ? m->cap_owned * 2 : 64;
        m->owned = (void**)realloc(m->owned, m->cap_owned * sizeof(void*));
    }
    m->owned[m->n_owned++] = p;
}

orc_model* orc_model_new(const orc_config* cfg) {
    h2f_table_init();
    orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
    m->cfg = *cfg;
    if (m->cfg.head_dim == 0 && m->cfg.num_heads) m->cfg.head_dim = m->cfg.hidden_size / m->cfg.num_heads;
    m->layers = (orc_layer*)calloc(cfg->num_layers ? cfg->num_layers : 1, sizeof(orc_layer));
    m->win_threshold = UINT32_MAX;
    return m;
}

void orc_model_set_window(orc_model* m, uint32_t window, uint32_t n_global, uint32_t threshold) {
    m->win = window;
    m->n_global = n_global;
    m->win_threshold = threshold;
}

void orc_model_free(orc_model* m) {
    if (!m) return;
    for (size_t i = 0; i < m->n_owned; ++i) free(m->owned[i]);
    free(m->owned);
    free(m->layers);
    orc_gguf_close(m->gguf);
    free(m);
}

void orc_model_config(const orc_model* m, orc_config* cfg) { *cfg = m->cfg; }

static float* to_f32_copy(orc_model* m, const void* data, int dtype, uint64_t n) {
    float* f = (float*)malloc(n * sizeof(float));
    for (uint64_t i = 0; i < n; ++i)
        f[i] = dtype == ORC_F16 ? orc_h2f(((const uint16_t*)data)[i]) : ((const float*)data)[i];
    own(m, f);
    return f;
}

static uint64_t expected_elems(const orc_config* c, const char* suffix) {
    uint64_t d = c->hidden_size, hd = c->head_dim, F = c->intermediate_size;
    if (!strcmp(suffix, "attn_q.weight")) return c->num_heads * hd * d;
    if (!strcmp(suffix, "attn_k.weight") || !strcmp(suffix, "attn_v.weight")) return c->num_kv_heads * hd * d;
    if (!strcmp(suffix, "attn_o.weight") || !strcmp(suffix, "attn_output.weight")) return d * c->num_heads * hd;
    if (!strcmp(suffix, "ffn_gate.weight") || !strcmp(suffix, "ffn_up.weight")) return F * d;
    if (!strcmp(suffix, "ffn_down.weight")) return d * F;
    if (!strcmp(suffix, "attn_norm.weight") || !strcmp(suffix, "ffn_norm.weight")) return d;
    return 0;
}

int orc_model_set_tensor(orc_model* m, const char* name, const void* data, int dtype, int copy) {
    const orc_config* c = &m->cfg;
    uint64_t d = c->hidden_size;
    if (!strcmp(name, "token_embd.weight") || !strcmp(name, "output.weight")) {
        uint64_t n = (uint64_t)c->vocab_size * d;
        const void* p = data;
        if (copy) {
            size_t bytes = n * (dtype == ORC_F16 ? 2 : 4);
            void* q = malloc(bytes);
            memcpy(q, data, bytes);
            own(m, q);
            p = q;
        }
        wref* w = !strcmp(name, "output.weight") ? &m->output : &m->tok_embd;
        w->p = p;
        w->t = dtype;
        return 0;
    }
    if (!strcmp(name, "output_norm.weight")) {
        m->out_norm = to_f32_copy(m, data, dtype, d);
        return 0;
    }
    unsigned layer;
    int off = 0;
    if (sscanf(name, "blk.%u.%n", &layer, &off) != 1 || off == 0) return -30;
    if (layer >= c->num_layers) return -30;
    const char* suffix = name + off;
    uint64_t n = expected_elems(c, suffix);
    if (n == 0) return -30;
    orc_layer* L = &m->layers[layer];
    if (!strcmp(suffix, "attn_norm.weight")) { L->attn_norm = to_f32_copy(m, data, dtype, n); return 0; }
    if (!strcmp(suffix, "ffn_norm.weight")) { L->ffn_norm = to_f32_copy(m, data, dtype, n); return 0; }
    const void* p = data;
    if (copy) {
        size_t bytes = n * (dtype == ORC_F16 ? 2 : 4);
        void* q = malloc(bytes);
        memcpy(q, data, bytes);
        own(m, q);
        p = q;
    }
    wref w = {p, dtype};
    if (!strcmp(suffix, "attn_q.weight")) L->q = w;
    else if (!strcmp(suffix, "attn_k.weight")) L->k = w;
    else if (!strcmp(suffix, "attn_v.weight")) L->v = w;
    else if (!strcmp(suffix, "attn_o.weight") || !strcmp(suffix, "attn_output.weight")) L->o = w;
    else if (!strcmp(suffix, "ffn_gate.weight")) L->gate = w;
    else if (!strcmp(suffix, "ffn_up.weight")) L->up = w;
    else if (!strcmp(suffix, "ffn_down.weight")) L->down = w;
    return 0;
}

int orc_model_check(const orc_model* m) {
    if (!m->tok_embd.p) return -30;
    for (uint32_t l = 0; l < m->cfg.num_layers; ++l) {
        const orc_layer* L = &m->layers[l];
        if (!L->attn_norm || !L->ffn_norm || !L->q.p || !L->k.p || !L->v.p || !L->o.p || !L->gate.p ||
            !L->up.p || !L->down.p)
            return -30;
    }
    return 0;
}

int orc_model_from_gguf(const char* path, orc_model** out) {
    *out = NULL;
    orc_gguf* g;
    int rc = orc_gguf_open(path, &g);
    if (rc) return rc;
    orc_config cfg;
    orc_gguf_model_config(g, &cfg);
    if (!cfg.hidden_size || !cfg.num_heads || !cfg.num_layers || !cfg.vocab_size || !cfg.num_kv_heads ||
        cfg.hidden_size % cfg.num_heads || cfg.num_heads % cfg.num_kv_heads) {
        orc_gguf_close(g);
        return -3;
    }
    orc_model* m = orc_model_new(&cfg);
    m->gguf = g;
    for (uint64_t i = 0; i < g->n_tensors; ++i) {
        const gti* t = &g->tis[i];
        if (t->kind < 0 && !t->quant) continue;
        const void* p = tensor_ptr(g, t);
        if (!p) { orc_model_free(m); return -11; }
        if (t->quant) { /* dequant-on-load: an owned fp32 copy */
            float* f = (float*)malloc((t->n_elem ? t->n_elem : 1) * sizeof(float));
            own(m, f);
            if (orc_dequant(p, t->data_size, t->raw_type, g->convention, t->n_elem, f) != (int64_t)t->n_elem) {
                orc_model_free(m);
                return -11;
            }
            orc_model_set_tensor(m, t->name, f, ORC_F32, 0);
            continue;
        }
        orc_model_set_tensor(m, t->name, p, t->kind, 0);
    }
    if (orc_model_check(m)) { orc_model_free(m); return -30; }
    *out = m;
    return 0;
}

/* =========================================================================================
 * primitives
 * ========================================================================================= */

/* rms_norm.comp:24-34: y = x / sqrt(mean(x^2) + eps) * g */
void orc_rmsnorm(const float* x, const float* gamma, uint32_t n, float eps, float* y) {
    double ss = 0.0;
    for (uint32_t i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
    double var = ss / (double)n + (double)eps;
    double inv = 1.0 / sqrt(var);
    for (uint32_t i = 0; i < n; ++i) y[i] = (float)((double)x[i] * inv * (double)(gamma ? gamma[i] : 1.0f));
}

/* Adjacent-pair rotary embedding (fused_matmul_rope.comp:48-81; frequencies Utils.cpp:101-110):
 * pair j = (2j, 2j+1), theta_j = base^(-2j/hd), angle = pos*theta_j,
 * (x, y) -> (x cos - y sin, x sin + y cos).  Angles in fp64. */
void orc_rope(float* v, uint32_t n_heads, uint32_t hd, uint32_t pos, float theta) {
    for (uint32_t j = 0; j < hd / 2; ++j) {
        double freq = pow((double)theta, -(double)(2 * j) / (double)hd);
        double ang = (double)pos * freq;
        float c = (float)cos(ang), s = (float)sin(ang);
        for (uint32_t h = 0; h < n_heads; ++h) {
            float* p = v + (size_t)h * hd + 2 * j;
            float x = p[0], y = p[1];
            p[0] = x * c - y * s;
            p[1] = x * s + y * c;
        }
    }
}

static void rope_cs(uint32_t hd, uint32_t pos, float theta, float* c, float* s) {
    for (uint32_t j = 0; j < hd / 2; ++j) {
        double freq = pow((double)theta, -(double)(2 * j) / (double)hd);
        double ang = (double)pos * freq;
        c[j] = (float)cos(ang);
        s[j] = (float)sin(ang);
    }
}

static void rope_apply(float* v, uint32_t n_heads, uint32_t hd, const float* c, const float* s) {
    for (uint32_t h = 0; h < n_heads; ++h)
        for (uint32_t j = 0; j < hd / 2; ++j) {
            float* p = v + (size_t)h * hd + 2 * j;
            float x = p[0], y = p[1];
            p[0] = x * c[j] - y * s[j];
            p[1] = x * s[j] + y * c[j];
        }
}

#if defined(__x86_64__)
__attribute__((target("avx2,fma,f16c"))) static double dot_f16_avx2(const uint16_t* w, const float* x, uint64_t K) {
    __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps(), a2 = _mm256_setzero_ps(), a3 = _mm256_setzero_ps();
    uint64_t k = 0;
    for (; k + 32 <= K; k += 32) {
        __m256 w0 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(w + k)));
        __m256 w1 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(w + k + 8)));
        __m256 w2 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(w + k + 16)));
        __m256 w3 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(w + k + 24)));
        a0 = _mm256_fmadd_ps(w0, _mm256_loadu_ps(x + k), a0);
        a1 = _mm256_fmadd_ps(w1, _mm256_loadu_ps(x + k + 8), a1);
        a2 = _mm256_fmadd_ps(w2, _mm256_loadu_ps(x + k + 16), a2);
        a3 = _mm256_fmadd_ps(w3, _mm256_loadu_ps(x + k + 24), a3);
    }
    float t[32];
    _mm256_storeu_ps(t, a0); _mm256_storeu_ps(t + 8, a1); _mm256_storeu_ps(t + 16, a2); _mm256_storeu_ps(t + 24, a3);
    double s = 0.0;
    for (int i = 0; i < 32; ++i) s += t[i];
    for (; k < K; ++k) s += (double)g_h2f_table[w[k]] * x[k];
    return s;
}
__attribute__((target("avx2,fma"))) static double dot_f32_avx2(const float* w, const float* x, uint64_t K) {
    __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps(), a2 = _mm256_setzero_ps(), a3 = _mm256_setzero_ps();
    uint64_t k = 0;
    for (; k + 32 <= K; k += 32) {
        a0 = _mm256_fmadd_ps(_mm256_loadu_ps(w + k), _mm256_loadu_ps(x + k), a0);
        a1 = _mm256_fmadd_ps(_mm256_loadu_ps(w + k + 8), _mm256_loadu_ps(x + k + 8), a1);
        a2 = _mm256_fmadd_ps(_mm256_loadu_ps(w + k + 16), _mm256_loadu_ps(x + k + 16), a2);
        a3 = _mm256_fmadd_ps(_mm256_loadu_ps(w + k + 24), _mm256_loadu_ps(x + k + 24), a3);
    }
    float t[32];
    _mm256_storeu_ps(t, a0); _mm256_storeu_ps(t + 8, a1); _mm256_storeu_ps(t + 16, a2); _mm256_storeu_ps(t + 24, a3);
    double s = 0.0;
    for (int i = 0; i < 32; ++i) s += t[i];
    for (; k < K; ++k) s += (double)w[k] * x[k];
    return s;
}
#endif

static int g_have_avx2 = -1;

static double dot_row(const wref* W, uint64_t row, uint64_t K, const float* x) {
#if defined(__x86_64__)
    if (g_have_avx2 < 0)
        g_have_avx2 = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") && __builtin_cpu_supports("f16c");
    if (g_have_avx2) {
        if (W->t == ORC_F16) return dot_f16_avx2((const uint16_t*)W->p + row * K, x, K);
        return dot_f32_avx2((const float*)W->p + row * K, x, K);
    }
#endif
    double s = 0.0;
    if (W->t == ORC_F16) {
        const uint16_t* w = (const uint16_t*)W->p + row * K;
        for (uint64_t k = 0; k < K; ++k) s += (double)g_h2f_table[w[k]] * (double)x[k];
    } else {
        const float* w = (const float*)W->p + row * K;
        for (uint64_t k = 0; k < K; ++k) s += (double)w[k] * (double)x[k];
    }
    return s;
}

/* y[o] = sum_i W[o*K+i] x[i]  (GGUF ne0 = input dim; final_linear.comp:63, feed_forward.comp:45) */
static void gemv(const wref* W, uint64_t N, uint64_t K, const float* x, float* y) {
    h2f_table_init();
    if (g_have_avx2 < 0) (void)dot_row(W, 0, 0, x);
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < (int64_t)N; ++o) y[o] = (float)dot_row(W, (uint64_t)o, K, x);
}

void orc_gemm_nt(const void* Wp, int wtype, uint32_t N, uint32_t K, const float* X, uint32_t B, float* Y) {
    h2f_table_init();
    wref W = {Wp, wtype};
    float* xc = (float*)malloc((size_t)K * sizeof(float));
    float* yc = (float*)malloc((size_t)N * sizeof(float));
    for (uint32_t b = 0; b < B; ++b) {
        for (uint32_t k = 0; k < K; ++k) xc[k] = X[(size_t)k * B + b];
        gemv(&W, N, K, xc, yc);
        for (uint32_t n = 0; n < N; ++n) Y[(size_t)n * B + b] = yc[n];
    }
    free(xc);
    free(yc);
}

/* attention.comp:92,116-189 for one query position, with KV read from the cache:
 * kv_head = head * n_kv / n_q; score = (q . k) * scale; softmax over positions 0..len-1;
 * out = sum_t p_t v_t.  fp64 accumulation. */
void orc_attention_decode(const float* q, const float* kc, const float* vc, uint32_t n_q,
                          uint32_t n_kv, uint32_t hd, uint32_t cap, uint32_t len, float scale,
                          float* out) {
    orc_attention_decode_window(q, kc, vc, n_q, n_kv, hd, cap, len, scale, 0, 0, UINT32_MAX, out);
}

/* Key k is attended by the query at position p = len - 1 when k <= p and, once len > threshold
 * (the reference switches to its sparse path when seq_len > 8192, VulkanSymbioteEngine.cpp:788),
 * when k < n_global (the global tokens) or k >= p - window (the sliding window,
 * sparse_attention.comp:84-85 window_start = pos - window_size).  The reference's shader takes
 * the contiguous range [min(global_end, window_start), ...) and clamps it to 1024-blocks
 * (:94-131), which drops the global tokens; that is not restated. */
static int window_keeps(uint32_t k, uint32_t len, uint32_t window, uint32_t n_global, uint32_t threshold) {
    const uint32_t p = len - 1;
    if (k > p) return 0;
    if (threshold == UINT32_MAX || len <= threshold) return 1;
    return k < n_global || (uint64_t)k + window >= p;
}

void orc_attention_decode_window(const float* q, const float* kc, const float* vc, uint32_t n_q,
                                 uint32_t n_kv, uint32_t hd, uint32_t cap, uint32_t len, float scale,
                                 uint32_t window, uint32_t n_global, uint32_t threshold, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t hh = 0; hh < (int64_t)n_q; ++hh) {
        uint32_t h = (uint32_t)hh;
        uint32_t kvh = (uint32_t)(((uint64_t)h * n_kv) / n_q);
        const float* qh = q + (size_t)h * hd;
        double* sc = (double*)malloc((size_t)len * sizeof(double));
        double mx = -INFINITY;
        for (uint32_t t = 0; t < len; ++t) {
            if (!window_keeps(t, len, window, n_global, threshold)) continue;
            const float* kt = kc + ((size_t)kvh * cap + t) * hd;
            double s = 0.0;
            for (uint32_t d = 0; d < hd; ++d) s += (double)qh[d] * (double)kt[d];
            s *= (double)scale;
            sc[t] = s;
            if (s > mx) mx = s;
        }
        double sum = 0.0;
        for (uint32_t t = 0; t < len; ++t) {
            sc[t] = window_keeps(t, len, window, n_global, threshold) ? exp(sc[t] - mx) : 0.0;
            sum += sc[t];
        }
        for (uint32_t d = 0; d < hd; ++d) {
            double acc = 0.0;
            for (uint32_t t = 0; t < len; ++t)
                if (sc[t] != 0.0) acc += sc[t] * (double)vc[((size_t)kvh * cap + t) * hd + d];
            out[(size_t)h * hd + d] = (float)(acc / sum);
        }
        free(sc);
    }
}

/* feed_forward.comp:21: silu(x) = x / (1 + exp(-x)); h = silu(gate) * up */
void orc_swiglu(const float* gate, const float* up, uint32_t n, float* h) {
    for (uint32_t i = 0; i < n; ++i) {
        double g = gate[i];
        h[i] = (float)(g / (1.0 + exp(-g)) * (double)up[i]);
    }
}

/* =========================================================================================
 * samplers
 * ========================================================================================= */
static uint32_t greedy(const float* l, uint32_t n) { /* VulkanSymbioteEngine.cpp:1794-1804 */
    uint32_t bi = 0;
    float bv = l[0];
    for (uint32_t i = 1; i < n; ++i)
        if (l[i] > bv) { bv = l[i]; bi = i; }
    return bi;
}

static const float* g_sort_logits;
static int cmp_desc(const void* a, const void* b) {
    uint32_t ia = *(const uint32_t*)a, ib = *(const uint32_t*)b;
    float la = g_sort_logits[ia], lb = g_sort_logits[ib];
    if (la > lb) return -1;
    if (la < lb) return 1;
    return ia < ib ? -1 : (ia > ib);
}

/* Uniform in [0,1) for sampling step `step`: Philox4x32-10 with key (seed, "sampler") and
 * counter (step, 0, 0, 0); 24 high bits of word 0. */
static float sample_uniform(uint64_t seed, uint64_t step) {
    uint32_t key[2], ctr[4] = {(uint32_t)step, (uint32_t)(step >> 32), 0, 0}, r[4];
    derive_key(seed, "sampler", key);
    orc_philox4x32_10(ctr, key, r);
    return (float)(r[0] >> 8) * (1.0f / 16777216.0f);
}

uint32_t orc_sample(const float* logits, uint32_t n, int sampler, float temperature, uint32_t top_k,
                    uint64_t seed, uint64_t step) {
    if (sampler == ORC_SAMPLE_GREEDY || temperature <= 0.0f) return greedy(logits, n);
    if (sampler == ORC_SAMPLE_REFERENCE) {
        /* member top_k_sampling (:1806-1855): logits/T, softmax, first index of the max prob */
        float* w = (float*)malloc((size_t)n * sizeof(float));
        for (uint32_t i = 0; i < n; ++i) w[i] = temperature != 1.0f ? logits[i] / temperature : logits[i];
        float mx = w[0];
        for (uint32_t i = 1; i < n; ++i) if (w[i] > mx) mx = w[i];
        float sum = 0.0f;
        for (uint32_t i = 0; i < n; ++i) { w[i] = expf(w[i] - mx); sum += w[i]; }
        for (uint32_t i = 0; i < n; ++i) w[i] /= sum;
        uint32_t r = greedy(w, n);
        free(w);
        return r;
    }
    /* Utils.cpp:140-172 with a reproducible uniform; ties in the partial sort -> lower id first */
    uint32_t k = top_k == 0 || top_k > n ? n : top_k;
    uint32_t* idx = (uint32_t*)malloc((size_t)n * sizeof(uint32_t));
    for (uint32_t i = 0; i < n; ++i) idx[i] = i;
    g_sort_logits = logits;
    qsort(idx, n, sizeof(uint32_t), cmp_desc);
    float* w = (float*)malloc((size_t)k * sizeof(float));
    float mx = logits[idx[0]], sum = 0.0f;
    for (uint32_t i = 0; i < k; ++i) { w[i] = expf((logits[idx[i]] - mx) / temperature); sum += w[i]; }
    for (uint32_t i = 0; i < k; ++i) w[i] /= sum;
    float r = sample_uniform(seed, step), cum = 0.0f;
    uint32_t pick = idx[0];
    for (uint32_t i = 0; i < k; ++i) {
        cum += w[i];
        if (r < cum) { pick = idx[i]; break; }
    }
    free(w);
    free(idx);
    return pick;
}

/* =========================================================================================
 * decoding state + forward
 * ========================================================================================= */
struct orc_state {
    orc_config cfg;
    uint32_t cap;
    int kv_f16;
    float** kc; /* per layer [n_kv][cap][hd] */
    float** vc;
    float *x, *n, *q, *k, *v, *o, *g, *u, *h, *tmp, *cs, *sn, *final;
};

orc_state* orc_state_new(const orc_model* m, uint32_t capacity, int kv_f16) {
    orc_state* s = (orc_state*)calloc(1, sizeof(orc_state));
    s->cfg = m->cfg;
    s->cap = capacity;
    s->kv_f16 = kv_f16;
    const orc_config* c = &m->cfg;
    size_t kvn = (size_t)c->num_kv_heads * capacity * c->head_dim;
    s->kc = (float**)calloc(c->num_layers, sizeof(float*));
    s->vc = (float**)calloc(c->num_layers, sizeof(float*));
    for (uint32_t l = 0; l < c->num_layers; ++l) {
        s->kc[l] = (float*)calloc(kvn, sizeof(float));
        s->vc[l] = (float*)calloc(kvn, sizeof(float));
        if (!s->kc[l] || !s->vc[l]) { orc_state_free(s); return NULL; }
    }
    size_t d = c->hidden_size, qd = (size_t)c->num_heads * c->head_dim, F = c->intermediate_size;
    s->x = (float*)calloc(d, 4); s->n = (float*)calloc(d, 4); s->q = (float*)calloc(qd, 4);
    s->k = (float*)calloc((size_t)c->num_kv_heads * c->head_dim, 4);
    s->v = (float*)calloc((size_t)c->num_kv_heads * c->head_dim, 4);
    s->o = (float*)calloc(qd, 4); s->g = (float*)calloc(F, 4); s->u = (float*)calloc(F, 4);
    s->h = (float*)calloc(F, 4); s->tmp = (float*)calloc(d > qd ? d : qd, 4);
    s->cs = (float*)calloc(c->head_dim, 4); s->sn = (float*)calloc(c->head_dim, 4);
    s->final = (float*)calloc(d, 4);
    return s;
}

void orc_state_free(orc_state* s) {
    if (!s) return;
    for (uint32_t l = 0; l < s->cfg.num_layers; ++l) {
        if (s->kc) free(s->kc[l]);
        if (s->vc) free(s->vc[l]);
    }
    free(s->kc); free(s->vc);
    free(s->x); free(s->n); free(s->q); free(s->k); free(s->v); free(s->o); free(s->g); free(s->u);
    free(s->h); free(s->tmp); free(s->cs); free(s->sn); free(s->final);
    free(s);
}

void orc_state_reset(orc_state* s) {
    size_t kvn = (size_t)s->cfg.num_kv_heads * s->cap * s->cfg.head_dim;
    for (uint32_t l = 0; l < s->cfg.num_layers; ++l) {
        memset(s->kc[l], 0, kvn * 4);
        memset(s->vc[l], 0, kvn * 4);
    }
}

const float* orc_state_last_hidden(const orc_state* s) { return s->final; }

int orc_forward(const orc_model* m, orc_state* s, uint32_t token, uint32_t pos, float* logits) {
    const orc_config* c = &m->cfg;
    if (pos >= s->cap) return -5;
    uint32_t d = c->hidden_size, hd = c->head_dim, nq = c->num_heads, nkv = c->num_kv_heads;
    uint32_t F = c->intermediate_size, V = c->vocab_size;
    uint32_t tok = token < V ? token : V - 1; /* embedding_lookup.comp:32 */
    if (m->tok_embd.t == ORC_F16) {
        const uint16_t* e = (const uint16_t*)m->tok_embd.p + (size_t)tok * d;
        for (uint32_t i = 0; i < d; ++i) s->x[i] = orc_h2f(e[i]);
    } else {
        memcpy(s->x, (const float*)m->tok_embd.p + (size_t)tok * d, (size_t)d * 4);
    }
    rope_cs(hd, pos, c->rope_theta, s->cs, s->sn);
    float scale = 1.0f / sqrtf((float)hd);
    for (uint32_t l = 0; l < c->num_layers; ++l) {
        const orc_layer* L = &m->layers[l];
        orc_rmsnorm(s->x, L->attn_norm, d, c->rms_eps, s->n);
        gemv(&L->q, (uint64_t)nq * hd, d, s->n, s->q);
        gemv(&L->k, (uint64_t)nkv * hd, d, s->n, s->k);
        gemv(&L->v, (uint64_t)nkv * hd, d, s->n, s->v);
        rope_apply(s->q, nq, hd, s->cs, s->sn);
        rope_apply(s->k, nkv, hd, s->cs, s->sn);
        for (uint32_t h = 0; h < nkv; ++h)
            for (uint32_t j = 0; j < hd; ++j) {
                float kv = s->k[h * hd + j], vv = s->v[h * hd + j];
                if (s->kv_f16) { kv = orc_h2f(orc_f2h(kv)); vv = orc_h2f(orc_f2h(vv)); }
                s->kc[l][((size_t)h * s->cap + pos) * hd + j] = kv;
                s->vc[l][((size_t)h * s->cap + pos) * hd + j] = vv;
            }
        orc_attention_decode_window(s->q, s->kc[l], s->vc[l], nq, nkv, hd, s->cap, pos + 1, scale, m->win,
                                    m->n_global, m->win_threshold, s->o);
        gemv(&L->o, d, (uint64_t)nq * hd, s->o, s->tmp);
        for (uint32_t i = 0; i < d; ++i) s->x[i] += s->tmp[i];
        orc_rmsnorm(s->x, L->ffn_norm, d, c->rms_eps, s->n);
        gemv(&L->gate, F, d, s->n, s->g);
        gemv(&L->up, F, d, s->n, s->u);
        orc_swiglu(s->g, s->u, F, s->h);
        gemv(&L->down, d, F, s->h, s->tmp);
        for (uint32_t i = 0; i < d; ++i) s->x[i] += s->tmp[i];
    }
    if (m->out_norm)
        orc_rmsnorm(s->x, m->out_norm, d, c->rms_eps, s->final);
    else
        memcpy(s->final, s->x, (size_t)d * 4);
    if (logits) {
        const wref* out = m->output.p ? &m->output : &m->tok_embd; /* tied when output.weight is absent */
        gemv(out, V, d, s->final, logits);
    }
    return 0;
}

int orc_generate(const orc_model* m, const uint32_t* prompt, uint32_t n_prompt, uint32_t max_new,
                 int sampler, float temperature, uint32_t top_k, uint64_t seed, int stop_on_eos,
                 int kv_f16, uint32_t* out_tokens, float* out_logits) {
    if (n_prompt == 0) return -1;
    if (max_new == 0) return 0;
    uint32_t V = m->cfg.vocab_size;
    orc_state* s = orc_state_new(m, n_prompt + max_new, kv_f16);
    if (!s) return -5;
    float* logits = (float*)malloc((size_t)V * 4);
    int rc = 0;
    for (uint32_t i = 0; i < n_prompt && rc == 0; ++i)
        rc = orc_forward(m, s, prompt[i], i, i + 1 == n_prompt ? logits : NULL);
    int produced = 0;
    for (uint32_t t = 0; t < max_new && rc == 0; ++t) {
        uint32_t tok = orc_sample(logits, V, sampler, temperature, top_k, seed, t);
        out_tokens[t] = tok;
        if (out_logits) memcpy(out_logits + (size_t)t * V, logits, (size_t)V * 4);
        produced = (int)t + 1;
        if (stop_on_eos && (tok == 0 || tok == 2)) break; /* VulkanSymbioteEngine.cpp:747-749 */
        if (t + 1 < max_new) rc = orc_forward(m, s, tok, n_prompt + t, logits);
    }
    free(logits);
    orc_state_free(s);
    return rc ? rc : produced;
}

int orc_teacher_forced(const orc_model* m, const uint32_t* ids, uint32_t n, uint32_t n_out, int kv_f16,
                       float* out) {
    if (n == 0 || n_out > n) return -1;
    uint32_t V = m->cfg.vocab_size;
    orc_state* s = orc_state_new(m, n, kv_f16);
    if (!s) return -5;
    int rc = 0;
    for (uint32_t i = 0; i < n && rc == 0; ++i) {
        float* lg = i >= n - n_out ? out + (size_t)(i - (n - n_out)) * V : NULL;
        rc = orc_forward(m, s, ids[i], i, lg);
    }
    orc_state_free(s);
    return rc;
}
