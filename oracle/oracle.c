/*
 * oracle.c -- CPU restatement of hobby-rs's single-sequence decode path
 * (HobbyLM hobby-rs/src/{gguf,config,quant,ops,model,sample,lib}.rs).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the timed CPU
 * baseline.  Nothing in the product links or loads it.
 *
 * Floating-point contract: build with -ffp-contract=off and without
 * -ffast-math (Rust never contracts a*b+c).  Every FMA below is explicit,
 * exactly where the reference issues one (_mm256_fmadd_ps in quant.rs:58,
 * f32x8::mul_add in ops.rs:18-27).  exp/pow/sin/cos come from the C library,
 * as Rust's f32::exp / f64::powf / f64::cos do on linux-gnu.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <fcntl.h>
#include <immintrin.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK 32

static __thread char g_err[512];

static int fail(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return -1;
}

const char *orc_last_error(void) { return g_err; }

static int g_threads = 0;
void orc_set_threads(int n) {
    g_threads = n;
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#endif
}
int orc_get_threads(void) {
#ifdef _OPENMP
    return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
    return 1;
#endif
}

/* ======================================================================
 * gguf.rs
 * ====================================================================== */

/* gguf.rs:329-341 */
float orc_half_to_f32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1;
    int exp = (h >> 10) & 0x1f;
    float mant = (float)(h & 0x3ff);
    float val;
    if (exp == 0)
        val = mant * ldexpf(1.0f, -24);
    else if (exp == 0x1f)
        val = (h & 0x3ff) == 0 ? INFINITY : NAN;
    else
        val = (1.0f + mant / 1024.0f) * ldexpf(1.0f, exp - 15);
    return sign ? -val : val;
}

static float rd_half(const uint8_t *b, size_t i) {
    return orc_half_to_f32((uint16_t)(b[i] | (b[i + 1] << 8)));
}

/* gguf.rs:361-363 */
void orc_dequant_f16(const uint8_t *b, size_t n, float *y) {
    for (size_t i = 0; i < n; i++) y[i] = rd_half(b, i * 2);
}

/* gguf.rs:365-375: block = {f16 d; int8 q[32]}, value = q * d */
void orc_dequant_q8_0(const uint8_t *b, size_t n, float *y) {
    for (size_t blk = 0; blk < n / 32; blk++) {
        size_t o = blk * 34;
        float d = rd_half(b, o);
        for (int j = 0; j < 32; j++) y[blk * 32 + j] = (float)(int8_t)b[o + 2 + j] * d;
    }
}

/* gguf.rs:377-397: block {f16 d; u32 qh; u8 qs[16]}; 5-bit values offset by -16 */
void orc_dequant_q5_0(const uint8_t *b, size_t n, float *y) {
    for (size_t blk = 0; blk < n / 32; blk++) {
        size_t o = blk * 22;
        float d = rd_half(b, o);
        uint32_t qh = (uint32_t)b[o + 2] | ((uint32_t)b[o + 3] << 8) | ((uint32_t)b[o + 4] << 16) |
                      ((uint32_t)b[o + 5] << 24);
        const uint8_t *qs = b + o + 6;
        for (uint32_t j = 0; j < 16; j++) {
            uint8_t xh0 = (uint8_t)(((qh >> j) << 4) & 0x10);
            uint8_t xh1 = (uint8_t)((qh >> (j + 12)) & 0x10);
            int x0 = (int)((qs[j] & 0x0F) | xh0) - 16;
            int x1 = (int)((qs[j] >> 4) | xh1) - 16;
            y[blk * 32 + j] = (float)x0 * d;
            y[blk * 32 + 16 + j] = (float)x1 * d;
        }
    }
}

/* gguf.rs:399-408 */
static void scale_min_k4(size_t j, const uint8_t *sc, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = sc[j] & 63;
        *m = sc[j + 4] & 63;
    } else {
        *d = (uint8_t)((sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4));
        *m = (uint8_t)((sc[j + 4] >> 4) | ((sc[j] >> 6) << 4));
    }
}

/* gguf.rs:410-439: 256-element super blocks {f16 d, dmin; u8 scales[12]; u8 qs[128]} */
void orc_dequant_q4_k(const uint8_t *b, size_t n, float *y) {
    size_t yi = 0;
    for (size_t blk = 0; blk < n / 256; blk++) {
        size_t o = blk * 144;
        float d = rd_half(b, o), dmin = rd_half(b, o + 2);
        const uint8_t *scales = b + o + 4, *qs = b + o + 16;
        size_t is = 0, q = 0;
        for (int it = 0; it < 4; it++) {
            uint8_t sc1, m1, sc2, m2;
            scale_min_k4(is, scales, &sc1, &m1);
            float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
            scale_min_k4(is + 1, scales, &sc2, &m2);
            float d2 = d * (float)sc2, mm2 = dmin * (float)m2;
            for (int l = 0; l < 32; l++) y[yi++] = d1 * (float)(qs[q + l] & 0xF) - mm1;
            for (int l = 0; l < 32; l++) y[yi++] = d2 * (float)(qs[q + l] >> 4) - mm2;
            q += 32;
            is += 2;
        }
    }
}

/* gguf.rs:441-468: 256-element super blocks {u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d} */
void orc_dequant_q6_k(const uint8_t *b, size_t n, float *y) {
    for (size_t blk = 0; blk < n / 256; blk++) {
        size_t o = blk * 210;
        const uint8_t *ql = b + o, *qh = b + o + 128;
        const int8_t *sc = (const int8_t *)(b + o + 192);
        float d = rd_half(b, o + 208);
        size_t ybase = blk * 256;
        for (int half = 0; half < 2; half++) {
            size_t yb = ybase + half * 128, qlb = half * 64, qhb = half * 32, scb = half * 8;
            for (size_t l = 0; l < 32; l++) {
                size_t is = l / 16;
                int q1 = (int)((ql[qlb + l] & 0xF) | (((qh[qhb + l] >> 0) & 3) << 4)) - 32;
                int q2 = (int)((ql[qlb + l + 32] & 0xF) | (((qh[qhb + l] >> 2) & 3) << 4)) - 32;
                int q3 = (int)((ql[qlb + l] >> 4) | (((qh[qhb + l] >> 4) & 3) << 4)) - 32;
                int q4 = (int)((ql[qlb + l + 32] >> 4) | (((qh[qhb + l] >> 6) & 3) << 4)) - 32;
                y[yb + l] = d * (float)sc[scb + is + 0] * (float)q1;
                y[yb + l + 32] = d * (float)sc[scb + is + 2] * (float)q2;
                y[yb + l + 64] = d * (float)sc[scb + is + 4] * (float)q3;
                y[yb + l + 96] = d * (float)sc[scb + is + 6] * (float)q4;
            }
        }
    }
}

enum { T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 };
enum { M_U32, M_I32, M_F32, M_U64, M_BOOL, M_STR, M_ARRSTR, M_ARRI32, M_ARRF32, M_OTHER };

typedef struct {
    char *key;
    int kind;
    uint64_t u; /* U32 / U64 / BOOL payload */
    int32_t i;
    float f;
    char *s;
    size_t arr_n;
} meta_t;

typedef struct {
    char *name;
    uint32_t nd;
    uint64_t ne[8];
    uint32_t type;
    uint64_t offset;
} tinfo_t;

typedef struct {
    const uint8_t *map;
    size_t size;
    size_t data_start;
    meta_t *meta;
    size_t n_meta;
    tinfo_t *t;
    size_t n_t;
} gguf_t;

typedef struct {
    const uint8_t *b;
    size_t n, p;
    int bad;
} cur_t;

static const uint8_t *take(cur_t *c, size_t n) {
    if (c->bad || n > c->n - c->p) {
        c->bad = 1;
        return NULL;
    }
    const uint8_t *r = c->b + c->p;
    c->p += n;
    return r;
}
static uint64_t rdu(cur_t *c, size_t n) {
    const uint8_t *p = take(c, n);
    uint64_t v = 0;
    if (!p) return 0;
    for (size_t k = 0; k < n; k++) v |= (uint64_t)p[k] << (8 * k);
    return v;
}
static char *gstr(cur_t *c) {
    uint64_t n = rdu(c, 8);
    const uint8_t *p = take(c, (size_t)n);
    if (!p) return NULL;
    char *s = (char *)malloc((size_t)n + 1);
    memcpy(s, p, (size_t)n);
    s[n] = 0;
    return s;
}

/* gguf.rs:109-125 */
static int read_scalar(cur_t *c, uint32_t ty, meta_t *m) {
    switch (ty) {
    case T_U8: m->kind = M_U32; m->u = rdu(c, 1); break;
    case T_I8: m->kind = M_I32; m->i = (int8_t)rdu(c, 1); break;
    case T_U16: m->kind = M_U32; m->u = rdu(c, 2); break;
    case T_I16: m->kind = M_I32; m->i = (int16_t)rdu(c, 2); break;
    case T_U32: m->kind = M_U32; m->u = rdu(c, 4); break;
    case T_I32: m->kind = M_I32; m->i = (int32_t)rdu(c, 4); break;
    case T_F32: { uint32_t u = (uint32_t)rdu(c, 4); m->kind = M_F32; memcpy(&m->f, &u, 4); } break;
    case T_BOOL: m->kind = M_BOOL; m->u = rdu(c, 1) != 0; break;
    case T_STR: m->kind = M_STR; m->s = gstr(c); break;
    case T_U64: m->kind = M_U64; m->u = rdu(c, 8); break;
    case T_I64: m->kind = M_I32; m->i = (int32_t)rdu(c, 8); break;
    case T_F64: { uint64_t u = rdu(c, 8); double d; memcpy(&d, &u, 8); m->kind = M_F32; m->f = (float)d; } break;
    default: return fail("GGUF: unsupported metadata scalar type %u", ty);
    }
    return c->bad ? fail("GGUF: unexpected end of file") : 0;
}

/* gguf.rs:127-163 */
static int read_value(cur_t *c, uint32_t ty, meta_t *m) {
    if (ty != T_ARR) return read_scalar(c, ty, m);
    uint32_t at = (uint32_t)rdu(c, 4);
    uint64_t n = rdu(c, 8);
    if (c->bad) return fail("GGUF: unexpected end of file");
    m->arr_n = (size_t)n;
    if (at == T_STR) {
        m->kind = M_ARRSTR;
        for (uint64_t k = 0; k < n; k++) {
            char *s = gstr(c);
            if (!s) return fail("GGUF: unexpected end of file");
            free(s);
        }
    } else if (at == T_I32 || at == T_U32) {
        m->kind = M_ARRI32;
        if (!take(c, (size_t)n * 4)) return fail("GGUF: unexpected end of file");
    } else if (at == T_F32) {
        m->kind = M_ARRF32;
        if (!take(c, (size_t)n * 4)) return fail("GGUF: unexpected end of file");
    } else {
        m->kind = M_OTHER;
        for (uint64_t k = 0; k < n; k++) {
            meta_t tmp = {0};
            if (read_scalar(c, at, &tmp)) return -1;
            free(tmp.s);
        }
    }
    return 0;
}

static void gguf_close(gguf_t *g) {
    if (g->map) munmap((void *)g->map, g->size);
    for (size_t k = 0; k < g->n_meta; k++) { free(g->meta[k].key); free(g->meta[k].s); }
    for (size_t k = 0; k < g->n_t; k++) free(g->t[k].name);
    free(g->meta);
    free(g->t);
    memset(g, 0, sizeof *g);
}

/* Gguf::open, gguf.rs:166-212 */
static int gguf_open(const char *path, gguf_t *g) {
    memset(g, 0, sizeof *g);
    int fd = open(path, O_RDONLY);
    if (fd < 0) return fail("opening %s", path);
    struct stat st;
    if (fstat(fd, &st) != 0) { close(fd); return fail("opening %s", path); }
    g->size = (size_t)st.st_size;
    if (g->size == 0) { close(fd); return fail("GGUF: unexpected end of file"); }
    void *p = mmap(NULL, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (p == MAP_FAILED) return fail("mmap %s failed", path);
    g->map = (const uint8_t *)p;
    cur_t c = {g->map, g->size, 0, 0};
    uint32_t magic = (uint32_t)rdu(&c, 4);
    if (c.bad) { gguf_close(g); return fail("GGUF: unexpected end of file"); }
    if (magic != 0x46554747u) { gguf_close(g); return fail("not a GGUF file (bad magic)"); }
    uint32_t version = (uint32_t)rdu(&c, 4);
    if (c.bad) { gguf_close(g); return fail("GGUF: unexpected end of file"); }
    if (version != 3) { gguf_close(g); return fail("unsupported GGUF version %u (expected 3)", version); }
    uint64_t n_t = rdu(&c, 8), n_m = rdu(&c, 8);
    if (c.bad || n_t > g->size || n_m > g->size) { gguf_close(g); return fail("GGUF: unexpected end of file"); }
    g->meta = (meta_t *)calloc((size_t)n_m + 1, sizeof(meta_t));
    for (uint64_t k = 0; k < n_m; k++) {
        meta_t m = {0};
        m.key = gstr(&c);
        uint32_t ty = (uint32_t)rdu(&c, 4);
        if (c.bad || !m.key) { free(m.key); gguf_close(g); return fail("GGUF: unexpected end of file"); }
        if (read_value(&c, ty, &m)) { free(m.key); free(m.s); char e[512]; snprintf(e, sizeof e, "%s", g_err); gguf_close(g); return fail("%s", e); }
        /* HashMap::insert: a repeated key replaces the earlier value */
        size_t slot = g->n_meta;
        for (size_t q = 0; q < g->n_meta; q++)
            if (strcmp(g->meta[q].key, m.key) == 0) { slot = q; free(g->meta[q].key); free(g->meta[q].s); break; }
        g->meta[slot] = m;
        if (slot == g->n_meta) g->n_meta++;
    }
    g->t = (tinfo_t *)calloc((size_t)n_t + 1, sizeof(tinfo_t));
    for (uint64_t k = 0; k < n_t; k++) {
        tinfo_t t = {0};
        t.name = gstr(&c);
        t.nd = (uint32_t)rdu(&c, 4);
        if (c.bad || !t.name || t.nd > 8) { free(t.name); gguf_close(g); return fail("GGUF: unexpected end of file"); }
        for (uint32_t d = 0; d < t.nd; d++) t.ne[d] = rdu(&c, 8);
        t.type = (uint32_t)rdu(&c, 4);
        t.offset = rdu(&c, 8);
        if (c.bad) { free(t.name); gguf_close(g); return fail("GGUF: unexpected end of file"); }
        size_t slot = g->n_t;
        for (size_t q = 0; q < g->n_t; q++)
            if (strcmp(g->t[q].name, t.name) == 0) { slot = q; free(g->t[q].name); break; }
        g->t[slot] = t;
        if (slot == g->n_t) g->n_t++;
    }
    size_t align = 32;
    for (size_t q = 0; q < g->n_meta; q++)
        if (strcmp(g->meta[q].key, "general.alignment") == 0 && g->meta[q].kind == M_U32)
            align = (size_t)g->meta[q].u;
    if (align == 0) { gguf_close(g); return fail("GGUF: general.alignment is 0"); }
    g->data_start = (c.p + align - 1) / align * align;
    return 0;
}

static const meta_t *meta_get(const gguf_t *g, const char *key) {
    for (size_t q = 0; q < g->n_meta; q++)
        if (strcmp(g->meta[q].key, key) == 0) return &g->meta[q];
    return NULL;
}
/* gguf.rs:272-279 */
static int get_u32(const gguf_t *g, const char *key, uint32_t *v) {
    const meta_t *m = meta_get(g, key);
    if (!m) return 0;
    if (m->kind == M_U32 || m->kind == M_U64) { *v = (uint32_t)m->u; return 1; }
    if (m->kind == M_I32) { *v = (uint32_t)m->i; return 1; }
    return 0;
}
/* gguf.rs:280-286 */
static int get_f32(const gguf_t *g, const char *key, float *v) {
    const meta_t *m = meta_get(g, key);
    if (!m) return 0;
    if (m->kind == M_F32) { *v = m->f; return 1; }
    if (m->kind == M_U32) { *v = (float)(uint32_t)m->u; return 1; }
    return 0;
}
/* gguf.rs:287-292 */
static int get_bool(const gguf_t *g, const char *key, int *v) {
    const meta_t *m = meta_get(g, key);
    if (!m || m->kind != M_BOOL) return 0;
    *v = (int)m->u;
    return 1;
}
static const tinfo_t *tensor_get(const gguf_t *g, const char *name) {
    for (size_t q = 0; q < g->n_t; q++)
        if (strcmp(g->t[q].name, name) == 0) return &g->t[q];
    return NULL;
}
static uint64_t n_elems(const tinfo_t *t) {
    uint64_t n = 1;
    for (uint32_t d = 0; d < t->nd; d++)
        if (__builtin_mul_overflow(n, t->ne[d], &n)) return UINT64_MAX;
    return n;
}

/* Gguf::f32, gguf.rs:215-235: a copy of an F32 tensor (the reference lends a view). */
static float *gguf_f32(const gguf_t *g, const char *name, size_t *n_out) {
    const tinfo_t *t = tensor_get(g, name);
    if (!t) { fail("tensor `%s` not found in GGUF", name); return NULL; }
    if (t->type != 0) {
        fail("tensor `%s` is ggml_type %u (expected F32=0); this engine is F32-only for now", name, t->type);
        return NULL;
    }
    size_t n = (size_t)n_elems(t);
    if (n_elems(t) == UINT64_MAX || n > SIZE_MAX / 4) { fail("tensor `%s`: element count overflows", name); return NULL; }
    size_t off = g->data_start + (size_t)t->offset;
    if (off > g->size || n * 4 > g->size - off) { fail("tensor `%s` data out of bounds", name); return NULL; }
    if (off % 4) { fail("tensor `%s` is not 4-byte aligned", name); return NULL; }
    float *v = (float *)malloc(n * 4 + 4);
    memcpy(v, g->map + off, n * 4);
    *n_out = n;
    return v;
}

/* Gguf::load, gguf.rs:250-269, with type_nbytes (gguf.rs:349-359) */
static float *gguf_load(const gguf_t *g, const char *name, size_t *n_out) {
    const tinfo_t *t = tensor_get(g, name);
    if (!t) { fail("tensor `%s` not found", name); return NULL; }
    if (t->type == 0) return gguf_f32(g, name, n_out);
    size_t n = (size_t)n_elems(t), nbytes;
    if (n_elems(t) == UINT64_MAX || n > SIZE_MAX / 4) { fail("tensor `%s`: element count overflows", name); return NULL; }
    switch (t->type) {
    case 1: nbytes = n * 2; break;
    case 6: nbytes = (n / 32) * 22; break;
    case 8: nbytes = (n / 32) * 34; break;
    case 12: nbytes = (n / 256) * 144; break;
    case 14: nbytes = (n / 256) * 210; break;
    default: fail("type_nbytes: unsupported ggml_type %u", t->type); return NULL;   /* gguf.rs:358 */
    }
    size_t off = g->data_start + (size_t)t->offset;
    if (off > g->size || nbytes > g->size - off) { fail("tensor `%s` data out of bounds", name); return NULL; }
    float *v = (float *)calloc(n + 1, 4);
    const uint8_t *b = g->map + off;
    switch (t->type) {
    case 1: orc_dequant_f16(b, n, v); break;
    case 6: orc_dequant_q5_0(b, n, v); break;
    case 8: orc_dequant_q8_0(b, n, v); break;
    case 12: orc_dequant_q4_k(b, n, v); break;
    case 14: orc_dequant_q6_k(b, n, v); break;
    }
    *n_out = n;
    return v;
}

/* Gguf::open + Gguf::load (gguf.rs:166-212, 250-269) of one tensor; *n = element count, out
 * (NULL: count only) holds cap floats. */
int orc_gguf_load_tensor(const char *path, const char *name, float *out, uint64_t cap, uint64_t *n) {
    gguf_t g;
    if (gguf_open(path, &g)) return -1;
    size_t cnt = 0;
    float *v = gguf_load(&g, name, &cnt);
    int rc = 0;
    if (!v) rc = -1;
    else {
        *n = cnt;
        if (out) {
            if (cap < cnt) rc = fail("output too small");
            else memcpy(out, v, cnt * 4);
        }
        free(v);
    }
    gguf_close(&g);
    return rc;
}

/* ======================================================================
 * ops.rs
 * ====================================================================== */

float orc_expf(float x) { return expf(x); }

/* f32x8::reduce_add (wide 0.7.33, AVX): lo+hi, then movehl, then lane 0 + lane 1 --
 * the same sequence as the hsum in quant.rs:61-65. */
static inline float hsum8(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v);
    __m128 hi = _mm256_extractf128_ps(v, 1);
    __m128 s = _mm_add_ps(lo, hi);
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 0x01));
    return _mm_cvtss_f32(s);
}

/* ops.rs:7-36: four f32x8 FMA accumulators over 32-wide steps, an 8-wide tail on a0,
 * reduce ((a0+a1)+(a2+a3)), then a scalar tail without FMA. */
float orc_dot(const float *a, const float *b, size_t n) {
    __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
    size_t i = 0, main = n - n % 32;
    while (i < main) {
        a0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), a0);
        a1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 8), _mm256_loadu_ps(b + i + 8), a1);
        a2 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 16), _mm256_loadu_ps(b + i + 16), a2);
        a3 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 24), _mm256_loadu_ps(b + i + 24), a3);
        i += 32;
    }
    while (i + 8 <= n) {
        a0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), a0);
        i += 8;
    }
    float s = hsum8(_mm256_add_ps(_mm256_add_ps(a0, a1), _mm256_add_ps(a2, a3)));
    while (i < n) {
        s += a[i] * b[i];
        i++;
    }
    return s;
}

/* ops.rs:40-53 */
void orc_matvec_f32(const float *w, const float *x, float *y, size_t out, size_t in) {
#pragma omp parallel for schedule(static) if (out >= 64)
    for (size_t o = 0; o < out; o++) y[o] = orc_dot(w + o * in, x, in);
}

/* ops.rs:58-72 (each output element is dot(w_row, x_row), as in matvec) */
static void matmul_f32(const float *w, const float *x, float *y, size_t tn, size_t in, size_t out) {
#pragma omp parallel for schedule(static)
    for (size_t o = 0; o < out; o++)
        for (size_t t = 0; t < tn; t++) y[t * out + o] = orc_dot(w + o * in, x + t * in, in);
}

float orc_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
float orc_silu(float x) { return x * orc_sigmoid(x); }

/* ops.rs:85-96 */
void orc_rmsnorm(const float *x, const float *w, float eps, float *out, size_t n) {
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) ss += x[i] * x[i];
    float scale = 1.0f / sqrtf(ss / (float)n + eps);
    for (size_t i = 0; i < n; i++) out[i] = x[i] * scale * w[i];
}

/* model.rs:753-763 */
void orc_norm_head(float *v, const float *w, float eps, size_t n) {
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) ss += v[i] * v[i];
    float scale = 1.0f / sqrtf(ss / (float)n + eps);
    for (size_t i = 0; i < n; i++) v[i] = v[i] * scale * w[i];
}

/* ops.rs:112-128 */
void orc_softmax(float *x, size_t n) {
    float m = -INFINITY;
    for (size_t i = 0; i < n; i++)
        if (x[i] > m) m = x[i];
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - m);
        sum += x[i];
    }
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; i++) x[i] *= inv;
}

/* ops.rs:139-152: angles in f64, rounded to f32 */
void orc_rope_table(size_t head_dim, size_t max_pos, float theta, float *cos_t, float *sin_t) {
    size_t half = head_dim / 2;
    for (size_t p = 0; p < max_pos; p++)
        for (size_t i = 0; i < half; i++) {
            double inv_freq = pow((double)theta, -(2.0 * (double)i) / (double)head_dim);
            double ang = (double)p * inv_freq;
            cos_t[p * half + i] = (float)cos(ang);
            sin_t[p * half + i] = (float)sin(ang);
        }
}

/* ops.rs:155-166: rotate-half */
void orc_rope_apply(const float *cos_t, const float *sin_t, size_t head_dim, float *v, size_t pos) {
    size_t half = head_dim / 2, base = pos * half;
    for (size_t i = 0; i < half; i++) {
        float c = cos_t[base + i], s = sin_t[base + i];
        float x1 = v[i], x2 = v[half + i];
        v[i] = x1 * c - x2 * s;
        v[half + i] = x2 * c + x1 * s;
    }
}

/* sample.rs:53-63: strict '>' so the first maximum wins; NaN never wins. */
uint32_t orc_argmax(const float *logits, size_t n) {
    size_t best = 0;
    float bv = -INFINITY;
    for (size_t i = 0; i < n; i++)
        if (logits[i] > bv) { bv = logits[i]; best = i; }
    return (uint32_t)best;
}

/* ======================================================================
 * sample.rs
 * ====================================================================== */

/* Rng::next_u64 (sample.rs:10-17): xorshift64* on the state; Rng::new (sample.rs:6-8) clamps a
 * zero seed to 1. */
uint64_t orc_rng_next_u64(uint64_t *state) {
    uint64_t x = *state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *state = x;
    return x * 0x2545F4914F6CDD1DULL;
}

/* Rng::next_f32 (sample.rs:18-20): the top 24 bits over 2^24 (both steps exact). */
float orc_rng_next_f32(uint64_t *state) {
    return (float)(orc_rng_next_u64(state) >> 40) / (float)(1ull << 24);
}

typedef struct {
    float p;
    uint32_t i;
} prob_t;

/* The nucleus order: probability descending.  sample.rs:86 sorts with sort_unstable_by, whose
 * order among equal probabilities is unspecified; here equal probabilities keep ascending
 * token ids (the order a stable sort of the id-ordered list gives). */
static int prob_desc(const void *a, const void *b) {
    const prob_t *x = (const prob_t *)a, *y = (const prob_t *)b;
    if (x->p > y->p) return -1;
    if (x->p < y->p) return 1;
    return x->i < y->i ? -1 : x->i > y->i;
}

/* sample::sample (sample.rs:66-112): temperature softmax (v / temp, max, exp(v - m), a sum in id
 * order, p /= sum), then with 0 < top_p < 1 the nucleus (descending order, cumulative sum until
 * it reaches top_p, renormalized by the kept sum); one uniform draw r, the first entry whose
 * cumulative probability exceeds r, else the last.  temp <= 0: argmax. */
uint32_t orc_sample(const float *logits, size_t n, float temp, float top_p, uint64_t *state) {
    if (!(temp > 0.0f)) return orc_argmax(logits, n);
    prob_t *pr = (prob_t *)malloc(n * sizeof(prob_t));
    float m = -INFINITY;
    for (size_t i = 0; i < n; i++) {
        pr[i].p = logits[i] / temp;
        pr[i].i = (uint32_t)i;
        m = fmaxf(m, pr[i].p);
    }
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        pr[i].p = expf(pr[i].p - m);
        sum += pr[i].p;
    }
    for (size_t i = 0; i < n; i++) pr[i].p /= sum;
    size_t cut = n;
    if (top_p > 0.0f && top_p < 1.0f) {
        qsort(pr, n, sizeof(prob_t), prob_desc);
        float cum = 0.0f;
        for (size_t i = 0; i < n; i++) {
            cum += pr[i].p;
            if (cum >= top_p) {
                cut = i + 1;
                break;
            }
        }
        float s = -0.0f;   /* <f32 as Sum>::sum */
        for (size_t i = 0; i < cut; i++) s += pr[i].p;
        for (size_t i = 0; i < cut; i++) pr[i].p /= s;
    }
    const float r = orc_rng_next_f32(state);
    float cum = 0.0f;
    uint32_t pick = cut ? pr[cut - 1].i : 0u;
    for (size_t i = 0; i < cut; i++) {
        cum += pr[i].p;
        if (r < cum) {
            pick = pr[i].i;
            break;
        }
    }
    free(pr);
    return pick;
}

/* sample::gumbel_argmax (sample.rs:32-50): argmax_i of l_i / temp - ln(-ln(u_i)), one draw u_i
 * (clamped to [1e-9, 1 - 1e-9]) per finite logit in id order; temp <= 0: argmax. */
uint32_t orc_gumbel_argmax(const float *logits, size_t n, float temp, uint64_t *state) {
    if (!(temp > 0.0f)) return orc_argmax(logits, n);
    size_t best = 0;
    float bv = -INFINITY;
    const float lo = 1e-9f, hi = 1.0f - 1e-9f;
    for (size_t i = 0; i < n; i++) {
        const float l = logits[i];
        if (!isfinite(l)) continue;
        float u = orc_rng_next_f32(state);
        u = u < lo ? lo : u > hi ? hi : u;
        const float val = l / temp + -logf(-logf(u));
        if (val > bv) {
            bv = val;
            best = i;
        }
    }
    return (uint32_t)best;
}

/* ======================================================================
 * quant.rs
 * ====================================================================== */

/* One 32-block of activation or weight quantization (quant.rs:90-99 and 114-122):
 * d = amax/127; id = d > 0 ? 1/d : 0; q = clamp(round(x*id), -127, 127), with
 * round() = half away from zero (f32::round). */
static inline void quant_block(const float *blk, int8_t *q, float *d_out) {
    float amax = 0.0f;
    for (int j = 0; j < QK; j++) amax = fmaxf(amax, fabsf(blk[j]));
    float d = amax / 127.0f;
    float id = d > 0.0f ? 1.0f / d : 0.0f;
    *d_out = d;
    for (int j = 0; j < QK; j++) {
        float r = roundf(blk[j] * id);
        if (r != r) r = 0.0f; /* Rust's saturating `as i8` maps NaN to 0 */
        if (r < -127.0f) r = -127.0f;
        if (r > 127.0f) r = 127.0f;
        q[j] = (int8_t)r;
    }
}

void orc_q8_quantize(const float *w, size_t out, size_t in, float *scales, int8_t *qs) {
    size_t nb = in / QK;
#pragma omp parallel for schedule(static)
    for (size_t o = 0; o < out; o++)
        for (size_t b = 0; b < nb; b++)
            quant_block(w + o * in + b * QK, qs + o * in + b * QK, scales + o * nb + b);
}

void orc_quantize_act(const float *x, size_t n, int8_t *qx, float *dx) {
    for (size_t b = 0; b < n / QK; b++) quant_block(x + b * QK, qx + b * QK, dx + b);
}

/* quant.rs:44-67 -- the same intrinsic sequence: sign/maddubs/madd gives eight exact
 * int32 partial sums per block (lane j = bytes 4j..4j+3); each is converted and
 * FMA-accumulated with the f32 product sw*dx into lane j; one hsum at the end. */
float orc_qrow_dot(const int8_t *qw, const int8_t *qa, const float *sw, const float *dx, size_t nb) {
    const __m256i ones = _mm256_set1_epi16(1);
    __m256 accf = _mm256_setzero_ps();
    for (size_t b = 0; b < nb; b++) {
        __m256i w = _mm256_loadu_si256((const __m256i *)(qw + b * QK));
        __m256i a = _mm256_loadu_si256((const __m256i *)(qa + b * QK));
        __m256i axw = _mm256_sign_epi8(w, w);
        __m256i say = _mm256_sign_epi8(a, w);
        __m256i p16 = _mm256_maddubs_epi16(axw, say);
        __m256i p32 = _mm256_madd_epi16(p16, ones);
        __m256 d = _mm256_set1_ps(sw[b] * dx[b]);
        accf = _mm256_fmadd_ps(d, _mm256_cvtepi32_ps(p32), accf);
    }
    return hsum8(accf);
}

/* quant.rs:106-136 */
void orc_q8_matvec(const float *scales, const int8_t *qs, size_t out, size_t in,
                   const float *x, float *y) {
    size_t nb = in / QK;
    int8_t *qx = (int8_t *)malloc(in + 32);
    float *dx = (float *)malloc(nb * 4 + 4);
    orc_quantize_act(x, in, qx, dx);
#pragma omp parallel for schedule(static) if (out >= 64)
    for (size_t o = 0; o < out; o++) y[o] = orc_qrow_dot(qs + o * in, qx, scales + o * nb, dx, nb);
    free(qx);
    free(dx);
}

/* quant.rs:144-194: scalar per-block integer dot, acc += (sw*dx)*isum in block order */
void orc_q8_matmul(const float *scales, const int8_t *qs, size_t out, size_t in,
                   const float *x, float *y, size_t tn) {
    size_t nb = in / QK;
    int8_t *qx = (int8_t *)malloc(tn * in + 32);
    float *dx = (float *)malloc(tn * nb * 4 + 4);
    for (size_t t = 0; t < tn; t++) orc_quantize_act(x + t * in, in, qx + t * in, dx + t * nb);
#pragma omp parallel for schedule(static)
    for (size_t o = 0; o < out; o++) {
        const int8_t *qw = qs + o * in;
        const float *sw = scales + o * nb;
        for (size_t t = 0; t < tn; t++) {
            const int8_t *qxr = qx + t * in;
            const float *dxr = dx + t * nb;
            float acc = 0.0f;
            for (size_t b = 0; b < nb; b++) {
                int32_t isum = 0;
                for (int j = 0; j < QK; j++) isum += (int32_t)qw[b * QK + j] * (int32_t)qxr[b * QK + j];
                acc += sw[b] * dxr[b] * (float)isum;
            }
            y[t * out + o] = acc;
        }
    }
    free(qx);
    free(dx);
}

/* ======================================================================
 * Mat (quant.rs:198-247)
 * ====================================================================== */

typedef struct {
    int q8;           /* 1: Q8Tensor, 0: owned F32 */
    size_t out, in;
    float *w;         /* F32 [out*in] */
    float *scales;    /* Q8 [out*in/32] */
    int8_t *qs;       /* Q8 [out*in] */
} mat_t;

static int mat_of(const float *w, size_t out, size_t in, int quant, mat_t *m) {
    memset(m, 0, sizeof *m);
    m->out = out;
    m->in = in;
    if (quant) {
        if (in % QK) return fail("Q8_0 needs in_ divisible by 32 (got %zu)", in);
        m->q8 = 1;
        m->scales = (float *)malloc(out * (in / QK) * 4 + 4);
        m->qs = (int8_t *)malloc(out * in + 32);
        orc_q8_quantize(w, out, in, m->scales, m->qs);
    } else {
        m->w = (float *)malloc(out * in * 4 + 4);
        memcpy(m->w, w, out * in * 4);
    }
    return 0;
}
static void mat_free(mat_t *m) {
    free(m->w);
    free(m->scales);
    free(m->qs);
}
static void mat_matvec(const mat_t *m, const float *x, float *y) {
    if (m->q8) orc_q8_matvec(m->scales, m->qs, m->out, m->in, x, y);
    else orc_matvec_f32(m->w, x, y, m->out, m->in);
}
static void mat_matmul(const mat_t *m, const float *x, float *y, size_t tn) {
    if (m->q8) orc_q8_matmul(m->scales, m->qs, m->out, m->in, x, y, tn);
    else matmul_f32(m->w, x, y, tn, m->in, m->out);
}
static size_t mat_bytes(const mat_t *m) {
    return m->q8 ? (m->out * m->in / QK) * 4 + m->out * m->in : m->out * m->in * 4;
}

/* ======================================================================
 * model.rs
 * ====================================================================== */

typedef struct {
    float *attn_norm, *q_norm, *k_norm, *ffn_norm;
    mat_t qkv, o;
    int moe;
    mat_t gate, up, down;           /* dense */
    mat_t router;                   /* F32 (n_exp, d) */
    float *bias;
    mat_t *gate_e, *up_e, *down_e;  /* per expert */
    mat_t gate_sh, up_sh, down_sh;
} layer_t;

struct orc_model {
    orc_config c;
    float *rope_cos, *rope_sin;
    float *token_embd;
    float *output_norm;
    mat_t output;
    layer_t *layers;
};

struct orc_kv {
    float **k, **v;    /* per layer [cap][kv_dim] */
    uint32_t cap, len, L, kvd;
    /* routing of the last processed row */
    uint32_t *r_idx;
    float *r_w, *r_gap;
    uint32_t top_k;
};

/* Config::from_gguf, config.rs:35-97 */
static int config_from_gguf(const gguf_t *g, orc_config *c) {
    memset(c, 0, sizeof *c);
    const meta_t *am = meta_get(g, "general.architecture");
    if (!am || am->kind != M_STR) return fail("missing general.architecture");
    const char *arch = am->s;
    char key[256];
#define K(s) (snprintf(key, sizeof key, "%s.%s", arch, s), key)
#define REQ(field, s) do { uint32_t v_; if (!get_u32(g, K(s), &v_)) return fail("missing metadata `%s.%s`", arch, s); c->field = v_; } while (0)
#define OPT(field, s, dflt) do { uint32_t v_; c->field = get_u32(g, K(s), &v_) ? v_ : (dflt); } while (0)
    uint32_t hd;
    if (get_u32(g, K("attention.key_length"), &hd)) c->head_dim = hd;
    else {
        uint32_t d = 0, h = 1;
        get_u32(g, K("embedding_length"), &d);
        get_u32(g, K("attention.head_count"), &h);
        c->head_dim = d / (h ? h : 1);
    }
    const tinfo_t *te = tensor_get(g, "token_embd.weight");
    uint32_t vs;
    if (te && te->nd > 1) c->vocab_size = (uint32_t)te->ne[1];
    else if (get_u32(g, K("vocab_size"), &vs)) c->vocab_size = vs;
    else return fail("cannot determine vocab_size");
    uint32_t gf;
    c->gating_sigmoid = get_u32(g, K("expert_gating_func"), &gf) ? (gf == 1 ? 0 : 1) : 1;
    REQ(d_model, "embedding_length");
    REQ(n_layers, "block_count");
    OPT(n_dense, "leading_dense_block_count", 1);
    REQ(n_heads, "attention.head_count");
    REQ(n_kv_heads, "attention.head_count_kv");
    REQ(dense_ffn, "feed_forward_length");
    REQ(expert_ffn, "expert_feed_forward_length");
    REQ(n_experts, "expert_count");
    REQ(top_k, "expert_used_count");
    OPT(n_shared, "expert_shared_count", 0);
    OPT(context_length, "context_length", 8192);
    if (!get_f32(g, K("attention.layer_norm_rms_epsilon"), &c->rms_eps)) c->rms_eps = 1e-5f;
    if (!get_f32(g, K("rope.freq_base"), &c->rope_theta)) c->rope_theta = 1e6f;
    if (!get_f32(g, K("expert_weights_scale"), &c->expert_weights_scale)) c->expert_weights_scale = 1.0f;
    int b;
    c->expert_weights_norm = get_bool(g, K("expert_weights_norm"), &b) ? b : 0;
    if (!get_u32(g, "diffusion.mask_token_id", &c->mask_token_id)) c->mask_token_id = 50257;
#undef K
#undef REQ
#undef OPT
    return 0;
}

static int shape_ok(size_t n, size_t want, const char *name) {
    if (n != want) return fail("tensor `%s` has %zu elements, expected %zu", name, n, want);
    return 0;
}

static float *load_norm(const gguf_t *g, const char *name, size_t want) {
    size_t n;
    float *v = gguf_f32(g, name, &n);
    if (v && shape_ok(n, want, name)) { free(v); return NULL; }
    return v;
}

static int load_mat(const gguf_t *g, const char *name, size_t out, size_t in, int quant, mat_t *m) {
    size_t n;
    float *w = gguf_load(g, name, &n);
    if (!w) return -1;
    if (shape_ok(n, out * in, name)) { free(w); return -1; }
    int r = mat_of(w, out, in, quant, m);
    free(w);
    return r;
}

/* split_experts, model.rs:17-21 */
static int load_experts(const gguf_t *g, const char *name, size_t ne, size_t a, size_t b, int quant, mat_t **out) {
    size_t n;
    float *w = gguf_load(g, name, &n);
    if (!w) return -1;
    if (shape_ok(n, ne * a * b, name)) { free(w); return -1; }
    mat_t *ms = (mat_t *)calloc(ne, sizeof(mat_t));
    for (size_t e = 0; e < ne; e++)
        if (mat_of(w + e * a * b, a, b, quant, &ms[e])) { free(w); return -1; }
    free(w);
    *out = ms;
    return 0;
}

void orc_model_free(orc_model *m) {
    if (!m) return;
    for (uint32_t i = 0; m->layers && i < m->c.n_layers; i++) {
        layer_t *L = &m->layers[i];
        free(L->attn_norm); free(L->q_norm); free(L->k_norm); free(L->ffn_norm); free(L->bias);
        mat_free(&L->qkv); mat_free(&L->o);
        mat_free(&L->gate); mat_free(&L->up); mat_free(&L->down); mat_free(&L->router);
        for (uint32_t e = 0; e < m->c.n_experts; e++) {
            if (L->gate_e) mat_free(&L->gate_e[e]);
            if (L->up_e) mat_free(&L->up_e[e]);
            if (L->down_e) mat_free(&L->down_e[e]);
        }
        free(L->gate_e); free(L->up_e); free(L->down_e);
        mat_free(&L->gate_sh); mat_free(&L->up_sh); mat_free(&L->down_sh);
    }
    free(m->layers);
    free(m->rope_cos); free(m->rope_sin); free(m->token_embd); free(m->output_norm);
    mat_free(&m->output);
    free(m);
}

/* Engine::load (lib.rs:85-92) + Model::load (model.rs:79-131).  The tokenizer is not
 * built (token ids cross the boundary), so its metadata keys are not required. */
int orc_model_load(const char *path, int quant, orc_model **out) {
    *out = NULL;
    gguf_t g;
    if (gguf_open(path, &g)) return -1;
    orc_model *m = (orc_model *)calloc(1, sizeof *m);
    if (config_from_gguf(&g, &m->c)) { gguf_close(&g); free(m); return -1; }
    orc_config *c = &m->c;
    size_t d = c->d_model, f = c->expert_ffn, hd = c->head_dim;
    size_t qd = (size_t)c->n_heads * hd, kvd = (size_t)c->n_kv_heads * hd;
    if (!d || !c->n_layers || !c->n_heads || !c->n_kv_heads || c->n_heads % c->n_kv_heads || hd % 2 ||
        c->top_k > c->n_experts || !c->context_length) {
        gguf_close(&g); free(m);
        return fail("unsupported hyperparameters");
    }
    m->rope_cos = (float *)malloc((size_t)c->context_length * hd / 2 * 4);
    m->rope_sin = (float *)malloc((size_t)c->context_length * hd / 2 * 4);
    orc_rope_table(hd, c->context_length, c->rope_theta, m->rope_cos, m->rope_sin);
    m->layers = (layer_t *)calloc(c->n_layers, sizeof(layer_t));
    char nm[256];
#define NM(s) (snprintf(nm, sizeof nm, "blk.%u.%s", i, s), nm)
    for (uint32_t i = 0; i < c->n_layers; i++) {
        layer_t *L = &m->layers[i];
        L->moe = i >= c->n_dense;
        if (L->moe) {
            size_t n;
            float *rw = gguf_load(&g, NM("ffn_gate_inp.weight"), &n);
            if (!rw || shape_ok(n, (size_t)c->n_experts * d, nm)) { free(rw); goto bad; }
            mat_of(rw, c->n_experts, d, 0, &L->router);
            free(rw);
            if (!(L->bias = load_norm(&g, NM("exp_probs_b.bias"), c->n_experts))) goto bad;
            if (load_experts(&g, NM("ffn_gate_exps.weight"), c->n_experts, f, d, quant, &L->gate_e)) goto bad;
            if (load_experts(&g, NM("ffn_up_exps.weight"), c->n_experts, f, d, quant, &L->up_e)) goto bad;
            if (load_experts(&g, NM("ffn_down_exps.weight"), c->n_experts, d, f, quant, &L->down_e)) goto bad;
            if (load_mat(&g, NM("ffn_gate_shexp.weight"), f, d, quant, &L->gate_sh)) goto bad;
            if (load_mat(&g, NM("ffn_up_shexp.weight"), f, d, quant, &L->up_sh)) goto bad;
            if (load_mat(&g, NM("ffn_down_shexp.weight"), d, f, quant, &L->down_sh)) goto bad;
        } else {
            if (load_mat(&g, NM("ffn_gate.weight"), c->dense_ffn, d, quant, &L->gate)) goto bad;
            if (load_mat(&g, NM("ffn_up.weight"), c->dense_ffn, d, quant, &L->up)) goto bad;
            if (load_mat(&g, NM("ffn_down.weight"), d, c->dense_ffn, quant, &L->down)) goto bad;
        }
        if (!(L->attn_norm = load_norm(&g, NM("attn_norm.weight"), d))) goto bad;
        if (load_mat(&g, NM("attn_qkv.weight"), qd + 2 * kvd, d, quant, &L->qkv)) goto bad;
        if (!(L->q_norm = load_norm(&g, NM("attn_q_norm.weight"), hd))) goto bad;
        if (!(L->k_norm = load_norm(&g, NM("attn_k_norm.weight"), hd))) goto bad;
        if (load_mat(&g, NM("attn_output.weight"), d, qd, quant, &L->o)) goto bad;
        if (!(L->ffn_norm = load_norm(&g, NM("ffn_norm.weight"), d))) goto bad;
    }
#undef NM
    if (load_mat(&g, "output.weight", c->vocab_size, d, quant, &m->output)) goto bad;
    {
        size_t n;
        m->token_embd = gguf_load(&g, "token_embd.weight", &n);
        if (!m->token_embd || shape_ok(n, (size_t)c->vocab_size * d, "token_embd.weight")) goto bad;
    }
    if (!(m->output_norm = load_norm(&g, "output_norm.weight", d))) goto bad;
    gguf_close(&g);
    *out = m;
    return 0;
bad: {
        char e[512];
        snprintf(e, sizeof e, "%s", g_err);
        gguf_close(&g);
        orc_model_free(m);
        return fail("%s", e);
    }
}

int orc_model_config(const orc_model *m, orc_config *cfg) {
    *cfg = m->c;
    return 0;
}

/* model.rs:134-149 */
uint64_t orc_weight_bytes(const orc_model *m) {
    uint64_t b = mat_bytes(&m->output);
    for (uint32_t i = 0; i < m->c.n_layers; i++) {
        const layer_t *L = &m->layers[i];
        b += mat_bytes(&L->qkv) + mat_bytes(&L->o);
        if (!L->moe) b += mat_bytes(&L->gate) + mat_bytes(&L->up) + mat_bytes(&L->down);
        else {
            for (uint32_t e = 0; e < m->c.n_experts; e++)
                b += mat_bytes(&L->gate_e[e]) + mat_bytes(&L->up_e[e]) + mat_bytes(&L->down_e[e]);
            b += mat_bytes(&L->gate_sh) + mat_bytes(&L->up_sh) + mat_bytes(&L->down_sh);
        }
    }
    return b;
}

/* KvCache::new, model.rs:67-74 */
int orc_kv_new(const orc_model *m, orc_kv **out) {
    orc_kv *kv = (orc_kv *)calloc(1, sizeof *kv);
    kv->L = m->c.n_layers;
    kv->kvd = m->c.n_kv_heads * m->c.head_dim;
    kv->cap = m->c.context_length;
    kv->k = (float **)calloc(kv->L, sizeof(float *));
    kv->v = (float **)calloc(kv->L, sizeof(float *));
    for (uint32_t l = 0; l < kv->L; l++) {
        kv->k[l] = (float *)malloc((size_t)kv->cap * kv->kvd * 4);
        kv->v[l] = (float *)malloc((size_t)kv->cap * kv->kvd * 4);
        if (!kv->k[l] || !kv->v[l]) { orc_kv_free(kv); return fail("KV cache allocation failed"); }
    }
    kv->top_k = m->c.top_k;
    kv->r_idx = (uint32_t *)malloc((size_t)kv->L * (kv->top_k + 1) * 4);
    kv->r_w = (float *)malloc((size_t)kv->L * (kv->top_k + 1) * 4);
    kv->r_gap = (float *)malloc((size_t)kv->L * 4);
    *out = kv;
    return 0;
}

void orc_kv_free(orc_kv *kv) {
    if (!kv) return;
    for (uint32_t l = 0; l < kv->L; l++) {
        if (kv->k) free(kv->k[l]);
        if (kv->v) free(kv->v[l]);
    }
    free(kv->k); free(kv->v); free(kv->r_idx); free(kv->r_w); free(kv->r_gap);
    free(kv);
}

uint32_t orc_kv_len(const orc_kv *kv) { return kv->len; }

int orc_kv_read(const orc_kv *kv, uint32_t layer, float *k, float *v) {
    if (layer >= kv->L) return fail("layer %u out of range", layer);
    memcpy(k, kv->k[layer], (size_t)kv->len * kv->kvd * 4);
    memcpy(v, kv->v[layer], (size_t)kv->len * kv->kvd * 4);
    return 0;
}

int orc_kv_load(orc_kv *kv, uint32_t len, const float *k, const float *v) {
    if (len > kv->cap) return fail("len %u exceeds cache capacity %u", len, kv->cap);
    size_t per = (size_t)len * kv->kvd;
    for (uint32_t l = 0; l < kv->L; l++) {
        memcpy(kv->k[l], k + l * per, per * 4);
        memcpy(kv->v[l], v + l * per, per * 4);
    }
    kv->len = len;
    return 0;
}

int orc_token_embedding(const orc_model *m, uint32_t id, float *out) {
    if (id >= m->c.vocab_size) return fail("token %u out of range (vocab %u)", id, m->c.vocab_size);
    memcpy(out, m->token_embd + (size_t)id * m->c.d_model, m->c.d_model * 4);
    return 0;
}

/* model.rs:212-233 on already normalised + rotated q; kc/vc hold n rows. */
static void attend(const orc_config *c, const float *q, const float *kc, const float *vc, size_t n,
                   float *out, float *scores) {
    size_t hd = c->head_dim, kvd = (size_t)c->n_kv_heads * hd, rep = c->n_heads / c->n_kv_heads;
    float scale = 1.0f / sqrtf((float)hd);
    memset(out, 0, (size_t)c->n_heads * hd * 4);
    for (size_t hq = 0; hq < c->n_heads; hq++) {
        size_t kvh = hq / rep;
        const float *qh = q + hq * hd;
        for (size_t t = 0; t < n; t++) scores[t] = orc_dot(qh, kc + t * kvd + kvh * hd, hd) * scale;
        orc_softmax(scores, n);
        float *oh = out + hq * hd;
        for (size_t t = 0; t < n; t++) {
            const float *vt = vc + t * kvd + kvh * hd;
            float p = scores[t];
            for (size_t di = 0; di < hd; di++) oh[di] += p * vt[di];
        }
    }
}

/* model.rs:199-208: QK-norm then RoPE on every q and k head */
static void qk_norm_rope(const orc_model *m, const layer_t *L, float *q, float *k, size_t pos) {
    const orc_config *c = &m->c;
    size_t hd = c->head_dim;
    for (size_t h = 0; h < c->n_heads; h++) {
        orc_norm_head(q + h * hd, L->q_norm, c->rms_eps, hd);
        orc_rope_apply(m->rope_cos, m->rope_sin, hd, q + h * hd, pos);
    }
    for (size_t h = 0; h < c->n_kv_heads; h++) {
        orc_norm_head(k + h * hd, L->k_norm, c->rms_eps, hd);
        orc_rope_apply(m->rope_cos, m->rope_sin, hd, k + h * hd, pos);
    }
}

void orc_attention_decode(float *q, float *k, const float *v, const float *q_norm,
                          const float *k_norm, const float *cos_t, const float *sin_t,
                          float eps, uint32_t n_heads, uint32_t n_kv, uint32_t hd,
                          uint32_t pos, float *kcache, float *vcache, float *out) {
    for (uint32_t h = 0; h < n_heads; h++) {
        orc_norm_head(q + (size_t)h * hd, q_norm, eps, hd);
        orc_rope_apply(cos_t, sin_t, hd, q + (size_t)h * hd, pos);
    }
    for (uint32_t h = 0; h < n_kv; h++) {
        orc_norm_head(k + (size_t)h * hd, k_norm, eps, hd);
        orc_rope_apply(cos_t, sin_t, hd, k + (size_t)h * hd, pos);
    }
    size_t kvd = (size_t)n_kv * hd;
    memcpy(kcache + (size_t)pos * kvd, k, kvd * 4);
    memcpy(vcache + (size_t)pos * kvd, v, kvd * 4);
    orc_config c = {0};
    c.n_heads = n_heads;
    c.n_kv_heads = n_kv;
    c.head_dim = hd;
    float *scores = (float *)malloc(((size_t)pos + 1) * 4);
    attend(&c, q, kcache, vcache, (size_t)pos + 1, out, scores);
    free(scores);
}

/* Model::attention, model.rs:186-238 */
static void attention(const orc_model *m, const layer_t *L, const float *h, uint32_t li, size_t pos,
                      orc_kv *kv, float *proj) {
    const orc_config *c = &m->c;
    size_t hd = c->head_dim, qd = (size_t)c->n_heads * hd, kvd = (size_t)c->n_kv_heads * hd;
    float *qkv = (float *)malloc((qd + 2 * kvd) * 4);
    mat_matvec(&L->qkv, h, qkv);
    float *q = qkv, *k = qkv + qd, *v = qkv + qd + kvd;
    qk_norm_rope(m, L, q, k, pos);
    memcpy(kv->k[li] + pos * kvd, k, kvd * 4);
    memcpy(kv->v[li] + pos * kvd, v, kvd * 4);
    float *out = (float *)malloc(qd * 4);
    float *scores = (float *)malloc((pos + 1) * 4);
    attend(c, q, kv->k[li], kv->v[li], pos + 1, out, scores);
    mat_matvec(&L->o, out, proj);
    free(qkv); free(out); free(scores);
}

/* Routing of one row (model.rs:270-293): returns top-k ids in rank order and weights. */
static void route(const orc_config *c, const float *logits, const float *bias, uint32_t *topk,
                  float *w, float *gap) {
    size_t ne = c->n_experts;
    float *scores = (float *)malloc(ne * 4), *sel = (float *)malloc(ne * 4);
    if (c->gating_sigmoid)
        for (size_t e = 0; e < ne; e++) scores[e] = orc_sigmoid(logits[e]);
    else {
        memcpy(scores, logits, ne * 4);
        orc_softmax(scores, ne);
    }
    for (size_t e = 0; e < ne; e++) sel[e] = scores[e] + bias[e];
    /* sort descending by sel; equal keys keep the lower index first */
    uint32_t *ord = (uint32_t *)malloc(ne * 4);
    for (size_t e = 0; e < ne; e++) ord[e] = (uint32_t)e;
    for (size_t a = 1; a < ne; a++) {
        uint32_t x = ord[a];
        size_t b = a;
        while (b > 0 && sel[ord[b - 1]] < sel[x]) { ord[b] = ord[b - 1]; b--; }
        ord[b] = x;
    }
    for (size_t r = 0; r < c->top_k; r++) { topk[r] = ord[r]; w[r] = scores[ord[r]]; }
    if (gap) *gap = c->top_k < ne ? sel[ord[c->top_k - 1]] - sel[ord[c->top_k]] : INFINITY;
    if (c->expert_weights_norm) {
        float s = 0.0f;
        for (size_t r = 0; r < c->top_k; r++) s += w[r];
        s += 1e-9f;
        for (size_t r = 0; r < c->top_k; r++) w[r] /= s;
    }
    free(scores); free(sel); free(ord);
}

int orc_route(const float *logits, const float *bias, uint32_t n_experts, uint32_t top_k,
              int gating_sigmoid, int weights_norm, uint32_t *idx, float *w, float *gap) {
    if (top_k == 0 || top_k > n_experts) return fail("top_k %u out of range", top_k);
    orc_config c = {0};
    c.n_experts = n_experts;
    c.top_k = top_k;
    c.gating_sigmoid = gating_sigmoid;
    c.expert_weights_norm = weights_norm;
    route(&c, logits, bias, idx, w, gap);
    return 0;
}

/* Model::ffn, model.rs:240-327 */
static void ffn(const orc_model *m, const layer_t *L, const float *h, float *out, orc_kv *kv, uint32_t li) {
    const orc_config *c = &m->c;
    size_t d = c->d_model;
    if (!L->moe) {
        size_t f = c->dense_ffn;
        float *g = (float *)malloc(f * 4), *u = (float *)malloc(f * 4);
        mat_matvec(&L->gate, h, g);
        mat_matvec(&L->up, h, u);
        for (size_t i = 0; i < f; i++) g[i] = orc_silu(g[i]) * u[i];
        mat_matvec(&L->down, g, out);
        free(g); free(u);
        for (uint32_t r = 0; r < c->top_k; r++) { kv->r_idx[li * c->top_k + r] = UINT32_MAX; kv->r_w[li * c->top_k + r] = 0; }
        kv->r_gap[li] = 0;
        return;
    }
    size_t f = c->expert_ffn, ne = c->n_experts;
    float *logits = (float *)malloc(ne * 4);
    mat_matvec(&L->router, h, logits);
    uint32_t *topk = kv->r_idx + (size_t)li * c->top_k;
    float *w = kv->r_w + (size_t)li * c->top_k;
    route(c, logits, L->bias, topk, w, &kv->r_gap[li]);
    memset(out, 0, d * 4);
    float *gb = (float *)malloc(f * 4), *ub = (float *)malloc(f * 4), *yb = (float *)malloc(d * 4);
    for (size_t r = 0; r < c->top_k; r++) {
        uint32_t e = topk[r];
        mat_matvec(&L->gate_e[e], h, gb);
        mat_matvec(&L->up_e[e], h, ub);
        for (size_t i = 0; i < f; i++) gb[i] = orc_silu(gb[i]) * ub[i];
        mat_matvec(&L->down_e[e], gb, yb);
        float scale = w[r] * c->expert_weights_scale;
        for (size_t i = 0; i < d; i++) out[i] += scale * yb[i];
    }
    if (c->n_shared > 0) {
        mat_matvec(&L->gate_sh, h, gb);
        mat_matvec(&L->up_sh, h, ub);
        for (size_t i = 0; i < f; i++) gb[i] = orc_silu(gb[i]) * ub[i];
        mat_matvec(&L->down_sh, gb, yb);
        for (size_t i = 0; i < d; i++) out[i] += yb[i];
    }
    free(logits); free(gb); free(ub); free(yb);
}

static int check_pos(const orc_model *m, const orc_kv *kv, uint32_t pos, uint32_t tn) {
    if (pos != kv->len) return fail("pos %u does not continue the cache (len %u)", pos, kv->len);
    if ((uint64_t)pos + tn > m->c.context_length)
        return fail("pos %u + %u exceeds context_length %u", pos, tn, m->c.context_length);
    return 0;
}

/* Model::forward_x, model.rs:160-184 */
int orc_forward_x(const orc_model *m, orc_kv *kv, const float *xin, uint32_t pos, float *logits) {
    if (check_pos(m, kv, pos, 1)) return -1;
    const orc_config *c = &m->c;
    size_t d = c->d_model;
    float *x = (float *)malloc(d * 4), *h = (float *)malloc(d * 4), *t = (float *)malloc(d * 4);
    memcpy(x, xin, d * 4);
    for (uint32_t li = 0; li < c->n_layers; li++) {
        const layer_t *L = &m->layers[li];
        orc_rmsnorm(x, L->attn_norm, c->rms_eps, h, d);
        attention(m, L, h, li, pos, kv, t);
        for (size_t i = 0; i < d; i++) x[i] += t[i];
        orc_rmsnorm(x, L->ffn_norm, c->rms_eps, h, d);
        ffn(m, L, h, t, kv, li);
        for (size_t i = 0; i < d; i++) x[i] += t[i];
    }
    kv->len = pos + 1;
    orc_rmsnorm(x, m->output_norm, c->rms_eps, h, d);
    float *lg = logits ? logits : (float *)malloc((size_t)c->vocab_size * 4);
    mat_matvec(&m->output, h, lg);
    if (!logits) free(lg);
    free(x); free(h); free(t);
    return 0;
}

/* Model::forward, model.rs:152-156 */
int orc_forward(const orc_model *m, orc_kv *kv, uint32_t token, uint32_t pos, float *logits) {
    if (token >= m->c.vocab_size) return fail("token %u out of range (vocab %u)", token, m->c.vocab_size);
    return orc_forward_x(m, kv, m->token_embd + (size_t)token * m->c.d_model, pos, logits);
}

/* Model::attn_prefill, model.rs:372-439 */
static void attn_prefill(const orc_model *m, const layer_t *L, const float *h, uint32_t li, size_t base,
                         size_t tn, orc_kv *kv, float *proj) {
    const orc_config *c = &m->c;
    size_t hd = c->head_dim, qd = (size_t)c->n_heads * hd, kvd = (size_t)c->n_kv_heads * hd;
    size_t qw = qd + 2 * kvd;
    float *qkv = (float *)malloc(tn * qw * 4);
    mat_matmul(&L->qkv, h, qkv, tn);
    for (size_t t = 0; t < tn; t++) qk_norm_rope(m, L, qkv + t * qw, qkv + t * qw + qd, base + t);
    for (size_t t = 0; t < tn; t++) {
        memcpy(kv->k[li] + (base + t) * kvd, qkv + t * qw + qd, kvd * 4);
        memcpy(kv->v[li] + (base + t) * kvd, qkv + t * qw + qd + kvd, kvd * 4);
    }
    float *o = (float *)malloc(tn * qd * 4);
#pragma omp parallel for schedule(static)
    for (size_t t = 0; t < tn; t++) {
        float *scores = (float *)malloc((base + t + 1) * 4);
        attend(c, qkv + t * qw, kv->k[li], kv->v[li], base + t + 1, o + t * qd, scores);
        free(scores);
    }
    mat_matmul(&L->o, o, proj, tn);
    free(qkv); free(o);
}

/* Model::ffn_prefill, model.rs:653-750 */
static void ffn_prefill(const orc_model *m, const layer_t *L, const float *h, size_t tn, float *out,
                        orc_kv *kv, uint32_t li) {
    const orc_config *c = &m->c;
    size_t d = c->d_model, f = c->expert_ffn;
    if (!L->moe) {
        size_t df = c->dense_ffn;
        float *g = (float *)malloc(tn * df * 4), *u = (float *)malloc(tn * df * 4);
        mat_matmul(&L->gate, h, g, tn);
        mat_matmul(&L->up, h, u, tn);
        for (size_t i = 0; i < tn * df; i++) g[i] = orc_silu(g[i]) * u[i];
        mat_matmul(&L->down, g, out, tn);
        free(g); free(u);
        for (uint32_t r = 0; r < c->top_k; r++) { kv->r_idx[li * c->top_k + r] = UINT32_MAX; kv->r_w[li * c->top_k + r] = 0; }
        kv->r_gap[li] = 0;
        return;
    }
    size_t ne = c->n_experts, k = c->top_k;
    float *logits = (float *)malloc(tn * ne * 4);
    mat_matmul(&L->router, h, logits, tn);
    /* assign[e] = list of (t, w) in token order */
    uint32_t *as_t = (uint32_t *)malloc(ne * tn * 4);
    float *as_w = (float *)malloc(ne * tn * 4);
    uint32_t *as_n = (uint32_t *)calloc(ne, 4);
    uint32_t *topk = (uint32_t *)malloc(k * 4);
    float *w = (float *)malloc(k * 4);
    for (size_t t = 0; t < tn; t++) {
        float gap;
        route(c, logits + t * ne, L->bias, topk, w, &gap);
        for (size_t r = 0; r < k; r++) {
            uint32_t e = topk[r];
            as_t[e * tn + as_n[e]] = (uint32_t)t;
            as_w[e * tn + as_n[e]] = w[r] * c->expert_weights_scale;
            as_n[e]++;
        }
        if (t == tn - 1) {
            memcpy(kv->r_idx + (size_t)li * k, topk, k * 4);
            memcpy(kv->r_w + (size_t)li * k, w, k * 4);
            kv->r_gap[li] = gap;
        }
    }
    memset(out, 0, tn * d * 4);
    for (size_t e = 0; e < ne; e++) {
        size_t mrow = as_n[e];
        if (!mrow) continue;
        float *xe = (float *)malloc(mrow * d * 4), *ge = (float *)malloc(mrow * f * 4);
        float *ue = (float *)malloc(mrow * f * 4), *ye = (float *)malloc(mrow * d * 4);
        for (size_t i = 0; i < mrow; i++) memcpy(xe + i * d, h + (size_t)as_t[e * tn + i] * d, d * 4);
        mat_matmul(&L->gate_e[e], xe, ge, mrow);
        mat_matmul(&L->up_e[e], xe, ue, mrow);
        for (size_t i = 0; i < mrow * f; i++) ge[i] = orc_silu(ge[i]) * ue[i];
        mat_matmul(&L->down_e[e], ge, ye, mrow);
        for (size_t i = 0; i < mrow; i++) {
            size_t t = as_t[e * tn + i];
            float wt = as_w[e * tn + i];
            for (size_t q = 0; q < d; q++) out[t * d + q] += wt * ye[i * d + q];
        }
        free(xe); free(ge); free(ue); free(ye);
    }
    if (c->n_shared > 0) {
        float *gs = (float *)malloc(tn * f * 4), *us = (float *)malloc(tn * f * 4), *ys = (float *)malloc(tn * d * 4);
        mat_matmul(&L->gate_sh, h, gs, tn);
        mat_matmul(&L->up_sh, h, us, tn);
        for (size_t i = 0; i < tn * f; i++) gs[i] = orc_silu(gs[i]) * us[i];
        mat_matmul(&L->down_sh, gs, ys, tn);
        for (size_t i = 0; i < tn * d; i++) out[i] += ys[i];
        free(gs); free(us); free(ys);
    }
    free(logits); free(as_t); free(as_w); free(as_n); free(topk); free(w);
}

/* Model::prefill, model.rs:340-370 */
int orc_prefill(const orc_model *m, orc_kv *kv, const float *inputs, uint32_t tn, float *logits) {
    if (tn == 0) return fail("prefill needs at least one input row");
    uint32_t base = kv->len;
    if (check_pos(m, kv, base, tn)) return -1;
    const orc_config *c = &m->c;
    size_t d = c->d_model;
    float *x = (float *)malloc((size_t)tn * d * 4), *h = (float *)malloc((size_t)tn * d * 4);
    float *t = (float *)malloc((size_t)tn * d * 4);
    memcpy(x, inputs, (size_t)tn * d * 4);
    for (uint32_t li = 0; li < c->n_layers; li++) {
        const layer_t *L = &m->layers[li];
        for (size_t r = 0; r < tn; r++) orc_rmsnorm(x + r * d, L->attn_norm, c->rms_eps, h + r * d, d);
        attn_prefill(m, L, h, li, base, tn, kv, t);
        for (size_t i = 0; i < (size_t)tn * d; i++) x[i] += t[i];
        for (size_t r = 0; r < tn; r++) orc_rmsnorm(x + r * d, L->ffn_norm, c->rms_eps, h + r * d, d);
        ffn_prefill(m, L, h, tn, t, kv, li);
        for (size_t i = 0; i < (size_t)tn * d; i++) x[i] += t[i];
    }
    kv->len = base + tn;
    float *hl = (float *)malloc(d * 4);
    orc_rmsnorm(x + (size_t)(tn - 1) * d, m->output_norm, c->rms_eps, hl, d);
    float *lg = logits ? logits : (float *)malloc((size_t)c->vocab_size * 4);
    mat_matvec(&m->output, hl, lg);
    if (!logits) free(lg);
    free(x); free(h); free(t); free(hl);
    return 0;
}

int orc_last_routing(const orc_kv *kv, uint32_t *idx, float *weight, float *gap) {
    size_t n = (size_t)kv->L * kv->top_k;
    if (idx) memcpy(idx, kv->r_idx, n * 4);
    if (weight) memcpy(weight, kv->r_w, n * 4);
    if (gap) memcpy(gap, kv->r_gap, (size_t)kv->L * 4);
    return 0;
}

/* Model::run_block (model.rs:471-508) with attn_block_cached (model.rs:512-585): the b block rows
 * (residual inputs) at positions base .. base + b - 1 attend to the cache's rows 0 .. base - 1
 * and to every block row (bidirectional within the block); the cache rows are not changed.
 * logits [b][V] (output.matmul), bk / bv [L][b][kv_dim] when not NULL.  The routing records of
 * kv take the block's last row. */
int orc_run_block(const orc_model *m, orc_kv *kv, const float *block, uint32_t b, uint32_t base, float *logits,
                  float *bk, float *bv) {
    if (b == 0) return fail("run_block needs at least one row");
    if (base > kv->len) return fail("base %u beyond the cache (len %u)", base, kv->len);
    const orc_config *c = &m->c;
    size_t d = c->d_model, hd = c->head_dim, qd = (size_t)c->n_heads * hd, kvd = (size_t)c->n_kv_heads * hd;
    size_t qw = qd + 2 * kvd, n = (size_t)base + b;
    float *x = (float *)malloc((size_t)b * d * 4), *h = (float *)malloc((size_t)b * d * 4);
    float *t = (float *)malloc((size_t)b * d * 4), *qkv = (float *)malloc((size_t)b * qw * 4);
    float *o = (float *)malloc((size_t)b * qd * 4);
    float *ka = (float *)malloc(n * kvd * 4), *va = (float *)malloc(n * kvd * 4);
    memcpy(x, block, (size_t)b * d * 4);
    for (uint32_t li = 0; li < c->n_layers; li++) {
        const layer_t *L = &m->layers[li];
        for (size_t r = 0; r < b; r++) orc_rmsnorm(x + r * d, L->attn_norm, c->rms_eps, h + r * d, d);
        mat_matmul(&L->qkv, h, qkv, b);
        for (size_t r = 0; r < b; r++) qk_norm_rope(m, L, qkv + r * qw, qkv + r * qw + qd, base + r);
        memcpy(ka, kv->k[li], (size_t)base * kvd * 4);
        memcpy(va, kv->v[li], (size_t)base * kvd * 4);
        for (size_t r = 0; r < b; r++) {
            memcpy(ka + (base + r) * kvd, qkv + r * qw + qd, kvd * 4);
            memcpy(va + (base + r) * kvd, qkv + r * qw + qd + kvd, kvd * 4);
            if (bk) memcpy(bk + ((size_t)li * b + r) * kvd, qkv + r * qw + qd, kvd * 4);
            if (bv) memcpy(bv + ((size_t)li * b + r) * kvd, qkv + r * qw + qd + kvd, kvd * 4);
        }
#pragma omp parallel for schedule(static)
        for (size_t r = 0; r < b; r++) {
            float *scores = (float *)malloc(n * 4);
            attend(c, qkv + r * qw, ka, va, n, o + r * qd, scores);
            free(scores);
        }
        mat_matmul(&L->o, o, t, b);
        for (size_t i = 0; i < (size_t)b * d; i++) x[i] += t[i];
        for (size_t r = 0; r < b; r++) orc_rmsnorm(x + r * d, L->ffn_norm, c->rms_eps, h + r * d, d);
        ffn_prefill(m, L, h, b, t, kv, li);
        for (size_t i = 0; i < (size_t)b * d; i++) x[i] += t[i];
    }
    if (logits) {
        for (size_t r = 0; r < b; r++) orc_rmsnorm(x + r * d, m->output_norm, c->rms_eps, h + r * d, d);
        mat_matmul(&m->output, h, logits, b);
    }
    free(x); free(h); free(t); free(qkv); free(o); free(ka); free(va);
    return 0;
}

/* Model::forward_bidir (model.rs:443-468): run_block over an empty prefix (attn_bidir,
 * model.rs:589-651, is attn_block_cached with base 0). */
int orc_forward_bidir(const orc_model *m, const float *inputs, uint32_t tn, float *logits) {
    orc_kv *kv;
    if (orc_kv_new(m, &kv)) return -1;
    int rc = orc_run_block(m, kv, inputs, tn, 0, logits, NULL, NULL);
    orc_kv_free(kv);
    return rc;
}

/* Engine::score_block (lib.rs:226-262), also the scoring of diffusion_block (lib.rs:167-205):
 * per row the ids >= valid masked, the presence penalty once per present id, the Gumbel pick,
 * softmax of the penalized row, the pick's probability and the current id's. */
static void score_rows(const orc_config *c, const float *all, size_t rows, size_t valid, const uint8_t *present,
                       float rp, float temp, uint64_t *rng, const uint32_t *cur, uint32_t *pred, float *pconf,
                       float *cconf) {
    size_t V = c->vocab_size;
    float *row = (float *)malloc(V * 4);
    for (size_t i = 0; i < rows; i++) {
        memcpy(row, all + i * V, V * 4);
        for (size_t l = valid; l < V; l++) row[l] = -INFINITY;
        if (rp != 1.0f)
            for (size_t t = 0; t < valid; t++)
                if (present[t]) row[t] = row[t] > 0.0f ? row[t] / rp : row[t] * rp;
        const uint32_t pk = orc_gumbel_argmax(row, V, temp, rng);
        orc_softmax(row, V);
        pred[i] = pk;
        pconf[i] = row[pk];
        cconf[i] = row[cur[i]];
    }
    free(row);
}

/* num_transfer (lib.rs:68-76) */
static void num_transfer(size_t n, size_t steps, size_t *out) {
    size_t base = n / steps;
    for (size_t i = 0; i < steps; i++) out[i] = base + (i < n - base * steps ? 1 : 0);
}

typedef struct {
    size_t i;
    float v;
} conf_t;
static int conf_desc(const void *a, const void *b) {   /* stable by index among equals */
    const conf_t *x = (const conf_t *)a, *y = (const conf_t *)b;
    if (x->v > y->v) return -1;
    if (x->v < y->v) return 1;
    return x->i < y->i ? -1 : x->i > y->i;
}
static int conf_asc(const void *a, const void *b) {
    const conf_t *x = (const conf_t *)a, *y = (const conf_t *)b;
    if (x->v < y->v) return -1;
    if (x->v > y->v) return 1;
    return x->i < y->i ? -1 : x->i > y->i;
}

/* The scoring of one block [b0, b0 + len) of ids `ids` (the canvas's, or the active block's):
 * cached: run_block of the block over the cache; uncached: forward_bidir of canvas[0 .. b0 + len). */
typedef struct {
    const orc_model *m;
    const orc_diff_opts *o;
    orc_kv *kv;           /* cached path: the persistent prefix cache */
    uint32_t *canvas;     /* uncached path: the whole canvas; cached: committed ids */
    size_t committed;     /* cached path: ids in canvas[] so far */
    uint64_t rng;
    size_t valid;
    uint32_t mask;
    float *all, *emb;
    uint8_t *present;
} diff_t;

static int diff_score(diff_t *D, const uint32_t *blk, size_t b0, size_t len, uint32_t *pred, float *pconf,
                      float *cconf) {
    const orc_config *c = &D->m->c;
    size_t d = c->d_model, V = c->vocab_size;
    memset(D->present, 0, D->valid);
    if (D->o->cached) {
        for (size_t i = 0; i < len; i++)
            if (orc_token_embedding(D->m, blk[i], D->emb + i * d)) return -1;
        if (orc_run_block(D->m, D->kv, D->emb, (uint32_t)len, (uint32_t)b0, D->all, NULL, NULL)) return -1;
        if (D->o->rep_penalty != 1.0f) {
            for (size_t i = 0; i < D->committed; i++)
                if (D->canvas[i] != D->mask && D->canvas[i] < D->valid) D->present[D->canvas[i]] = 1;
            for (size_t i = 0; i < len; i++)
                if (blk[i] != D->mask && blk[i] < D->valid) D->present[blk[i]] = 1;
        }
        score_rows(c, D->all, len, D->valid, D->present, D->o->rep_penalty, D->o->temp, &D->rng, blk, pred, pconf,
                   cconf);
    } else {
        size_t b1 = b0 + len;
        for (size_t i = 0; i < b1; i++)
            if (orc_token_embedding(D->m, D->canvas[i], D->emb + i * d)) return -1;
        if (orc_forward_bidir(D->m, D->emb, (uint32_t)b1, D->all)) return -1;
        if (D->o->rep_penalty != 1.0f)
            for (size_t i = 0; i < b1; i++)
                if (D->canvas[i] != D->mask && D->canvas[i] < D->valid) D->present[D->canvas[i]] = 1;
        score_rows(c, D->all + b0 * V, len, D->valid, D->present, D->o->rep_penalty, D->o->temp, &D->rng, blk, pred,
                   pconf, cconf);
    }
    return 0;
}

/* Engine::generate_diffusion (lib.rs:214-224): the prefix-cached (lib.rs:269-407) or the
 * uncached (lib.rs:410-495) semi-autoregressive denoising of gen_len ids after the prompt; the
 * generated ids up to the first eos in out_ids, their count in *n_out. */
int orc_generate_diffusion(const orc_model *m, const uint32_t *prompt, uint32_t n_prompt, const orc_diff_opts *o,
                           uint32_t eos, uint32_t *out_ids, uint32_t *n_out) {
    *n_out = 0;
    const orc_config *c = &m->c;
    size_t p = n_prompt, d = c->d_model, V = c->vocab_size, ctx = c->context_length;
    if (p == 0) return 0;
    if (o->block == 0 || o->steps == 0) return fail("block and steps must be positive");
    diff_t D;
    memset(&D, 0, sizeof D);
    D.m = m;
    D.o = o;
    D.rng = o->seed > 1 ? o->seed : 1;
    D.valid = V < 50257 ? V : 50257;
    D.mask = c->mask_token_id;
    size_t gen_len;
    if (o->cached) {
        size_t room = ctx > p + o->block ? ctx - (p + o->block) : 0;
        gen_len = o->gen_len < (room > 1 ? room : 1) ? o->gen_len : (room > 1 ? room : 1);
    } else {
        size_t room = ctx > p ? ctx - p : 0;
        gen_len = o->gen_len < (room > 1 ? room : 1) ? o->gen_len : (room > 1 ? room : 1);
    }
    size_t span = o->cached ? (o->block > p ? o->block : p) : p + gen_len;
    D.all = (float *)malloc(span * V * 4);
    D.emb = (float *)malloc(span * d * 4);
    D.present = (uint8_t *)malloc(D.valid);
    D.canvas = (uint32_t *)malloc((p + gen_len) * 4);
    memcpy(D.canvas, prompt, p * 4);
    uint32_t *blk = (uint32_t *)malloc(o->block * 4), *pred = (uint32_t *)malloc(o->block * 4);
    float *pconf = (float *)malloc(o->block * 4), *cconf = (float *)malloc(o->block * 4);
    conf_t *cand = (conf_t *)malloc(o->block * sizeof(conf_t));
    size_t *sched = NULL;
    int rc = 0;
    float *bk = NULL, *bv = NULL;
    size_t kvd = (size_t)c->n_kv_heads * c->head_dim, result = gen_len;
    if (o->cached) {
        if (orc_kv_new(m, &D.kv)) { rc = -1; goto out; }
        for (size_t i = 0; i < p; i++)
            if (orc_token_embedding(m, prompt[i], D.emb + i * d)) { rc = -1; goto out; }
        bk = (float *)malloc((size_t)c->n_layers * span * kvd * 4);
        bv = (float *)malloc((size_t)c->n_layers * span * kvd * 4);
        if (orc_run_block(m, D.kv, D.emb, (uint32_t)p, 0, NULL, bk, bv)) { rc = -1; goto out; }
        for (uint32_t li = 0; li < c->n_layers; li++) {
            memcpy(D.kv->k[li], bk + (size_t)li * p * kvd, p * kvd * 4);
            memcpy(D.kv->v[li], bv + (size_t)li * p * kvd, p * kvd * 4);
        }
        D.kv->len = (uint32_t)p;
        D.committed = p;
    } else {
        for (size_t i = p; i < p + gen_len; i++) D.canvas[i] = D.mask;
    }
    for (size_t b0 = p; b0 < p + gen_len;) {
        size_t b1 = b0 + o->block < p + gen_len ? b0 + o->block : p + gen_len, len = b1 - b0;
        uint32_t *cur = o->cached ? blk : D.canvas + b0;   /* the active block's ids */
        if (o->cached)
            for (size_t i = 0; i < len; i++) blk[i] = D.mask;
        if (o->cached && o->threshold > 0.0f) {   /* lib.rs:302-327 */
            for (size_t it = 0; it < (len > 1 ? len : 1); it++) {
                int anym = 0;
                for (size_t i = 0; i < len; i++) anym |= cur[i] == D.mask;
                if (!anym) break;
                if (diff_score(&D, cur, b0, len, pred, pconf, cconf)) { rc = -1; goto out; }
                int any = 0;
                size_t best = 0;
                float bvv = 0.0f;
                int have = 0;
                for (size_t i = 0; i < len; i++) {
                    if (cur[i] != D.mask) continue;
                    /* Iterator::max_by: the last of equal maxima */
                    if (!have || !(pconf[i] < bvv)) { best = i; bvv = pconf[i]; have = 1; }
                }
                for (size_t i = 0; i < len; i++)
                    if (cur[i] == D.mask && pconf[i] >= o->threshold) { cur[i] = pred[i]; any = 1; }
                if (!any) cur[best] = pred[best];
            }
        } else {   /* the num_transfer schedule (lib.rs:329-352, 428-451) */
            size_t sb = (size_t)roundf((float)(o->steps * len) / (float)gen_len);
            if (sb < 1) sb = 1;
            sched = (size_t *)realloc(sched, sb * sizeof(size_t));
            num_transfer(len, sb, sched);
            for (size_t s = 0; s < sb; s++) {
                if (diff_score(&D, cur, b0, len, pred, pconf, cconf)) { rc = -1; goto out; }
                size_t nc = 0;
                for (size_t i = 0; i < len; i++)
                    if (cur[i] == D.mask) { cand[nc].i = i; cand[nc].v = pconf[i]; nc++; }
                if (nc == 0) break;
                qsort(cand, nc, sizeof(conf_t), conf_desc);
                for (size_t q = 0; q < (sched[s] < nc ? sched[s] : nc); q++) cur[cand[q].i] = pred[cand[q].i];
            }
            int anym = 0;
            for (size_t i = 0; i < len; i++) anym |= cur[i] == D.mask;
            if (anym) {
                if (diff_score(&D, cur, b0, len, pred, pconf, cconf)) { rc = -1; goto out; }
                for (size_t i = 0; i < len; i++)
                    if (cur[i] == D.mask) cur[i] = pred[i];
            }
        }
        for (uint32_t rs = 0; rs < o->remask_steps; rs++) {   /* lib.rs:354-371, 453-468 */
            if (diff_score(&D, cur, b0, len, pred, pconf, cconf)) { rc = -1; goto out; }
            size_t r = (size_t)((float)len * o->remask_frac);
            if (r < 1) r = 1;
            for (size_t i = 0; i < len; i++) { cand[i].i = i; cand[i].v = cconf[i]; }
            qsort(cand, len, sizeof(conf_t), conf_asc);
            for (size_t q = 0; q < (r < len ? r : len); q++) cur[cand[q].i] = D.mask;
            if (diff_score(&D, cur, b0, len, pred, pconf, cconf)) { rc = -1; goto out; }
            for (size_t i = 0; i < len; i++)
                if (cur[i] == D.mask) cur[i] = pred[i];
        }
        if (o->cached) {   /* finalize: the block's K/V into the cache (lib.rs:374-381) */
            for (size_t i = 0; i < len; i++)
                if (orc_token_embedding(m, blk[i], D.emb + i * d)) { rc = -1; goto out; }
            if (orc_run_block(m, D.kv, D.emb, (uint32_t)len, (uint32_t)b0, NULL, bk, bv)) { rc = -1; goto out; }
            for (uint32_t li = 0; li < c->n_layers; li++) {
                memcpy(D.kv->k[li] + b0 * kvd, bk + (size_t)li * len * kvd, len * kvd * 4);
                memcpy(D.kv->v[li] + b0 * kvd, bv + (size_t)li * len * kvd, len * kvd * 4);
            }
            D.kv->len = (uint32_t)b1;
            memcpy(D.canvas + b0, blk, len * 4);
            D.committed = b1;
        }
        size_t endpos = b1;   /* the first eos of the generated region ends the generation */
        int hit = 0;
        for (size_t i = p; i < b1; i++)
            if (D.canvas[i] == eos) { endpos = i; hit = 1; break; }
        if (hit) { result = endpos - p; break; }
        b0 = b1;
    }
    memcpy(out_ids, D.canvas + p, result * 4);
    *n_out = (uint32_t)result;
out:
    if (D.kv) orc_kv_free(D.kv);
    free(D.all); free(D.emb); free(D.present); free(D.canvas); free(blk); free(pred); free(pconf); free(cconf);
    free(cand); free(sched); free(bk); free(bv);
    return rc;
}

/* Engine::generate (lib.rs:107-162): prefill, then per step the ids >= 50257 masked, the
 * repetition penalty once per earlier occurrence of a token, sample::sample with the seeded Rng
 * (lib.rs:115), a stop at eos or at the context length. */
int orc_generate(const orc_model *m, orc_kv *kv, const uint32_t *prompt, uint32_t n_prompt, uint32_t max_new,
                 float temp, float top_p, uint64_t seed, float rep_penalty, uint32_t eos, uint32_t *out_ids,
                 uint32_t *n_out) {
    *n_out = 0;
    if (n_prompt == 0) return 0;
    const orc_config *c = &m->c;
    size_t d = c->d_model, V = c->vocab_size;
    uint64_t rng = seed > 1 ? seed : 1;
    float *in = (float *)malloc((size_t)n_prompt * d * 4);
    for (uint32_t i = 0; i < n_prompt; i++)
        if (orc_token_embedding(m, prompt[i], in + (size_t)i * d)) { free(in); return -1; }
    float *logits = (float *)malloc(V * 4);
    uint32_t pos = n_prompt + kv->len;
    if (orc_prefill(m, kv, in, n_prompt, logits)) { free(in); free(logits); return -1; }
    free(in);
    size_t valid = V < 50257 ? V : 50257;
    uint32_t n = 0;
    for (uint32_t it = 0; it < max_new; it++) {
        for (size_t i = valid; i < V; i++) logits[i] = -INFINITY;
        if (rep_penalty != 1.0f)
            for (uint32_t q = 0; q < n; q++) {
                float *l = &logits[out_ids[q]];
                *l = *l > 0.0f ? *l / rep_penalty : *l * rep_penalty;
            }
        uint32_t next = orc_sample(logits, V, temp, top_p, &rng);
        if (next == eos) break;
        out_ids[n++] = next;
        if (pos + 1 >= c->context_length) break;
        if (orc_forward(m, kv, next, pos, logits)) { free(logits); *n_out = n; return -1; }
        pos++;
    }
    free(logits);
    *n_out = n;
    return 0;
}

/* Engine::generate (lib.rs:107-162) with temp = 0 (sample.rs:66-69 -> argmax). */
int orc_generate_greedy(const orc_model *m, orc_kv *kv, const uint32_t *prompt, uint32_t n_prompt,
                        uint32_t max_new, float rep_penalty, uint32_t eos, uint32_t *out_ids,
                        uint32_t *n_out) {
    *n_out = 0;
    if (n_prompt == 0) return 0;
    const orc_config *c = &m->c;
    size_t d = c->d_model, V = c->vocab_size;
    float *in = (float *)malloc((size_t)n_prompt * d * 4);
    for (uint32_t i = 0; i < n_prompt; i++)
        if (orc_token_embedding(m, prompt[i], in + (size_t)i * d)) { free(in); return -1; }
    float *logits = (float *)malloc(V * 4);
    uint32_t pos = n_prompt + kv->len;
    if (orc_prefill(m, kv, in, n_prompt, logits)) { free(in); free(logits); return -1; }
    free(in);
    size_t valid = V < 50257 ? V : 50257;
    uint32_t n = 0;
    for (uint32_t it = 0; it < max_new; it++) {
        for (size_t i = valid; i < V; i++) logits[i] = -INFINITY;
        if (rep_penalty != 1.0f)
            for (uint32_t q = 0; q < n; q++) {
                float *l = &logits[out_ids[q]];
                *l = *l > 0.0f ? *l / rep_penalty : *l * rep_penalty;
            }
        uint32_t next = orc_argmax(logits, V);
        if (next == eos) break;
        out_ids[n++] = next;
        if (pos + 1 >= c->context_length) break;
        if (orc_forward(m, kv, next, pos, logits)) { free(logits); *n_out = n; return -1; }
        pos++;
    }
    free(logits);
    *n_out = n;
    return 0;
}
