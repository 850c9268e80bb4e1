/* Synthetic DiT denoise step on the operator ABI (include/h3_dit_synth.h).
 *
 * The block body follows the reference's run_block op sequence
 * (src/denoise/dit.c:2286-2539): AdaLN (modulation slots 0/1) -> QKV projection
 * -> Q/K (RMSNorm and) RoPE split -> DiT attention -> output projection -> gate
 * (slot 2) fused with the second AdaLN (slots 3/4) -> MLP (GELU-tanh, or fc1 ->
 * SwiGLU -> fc2 as dit.c:2479-2485) -> gate (slot 5). The block loop and
 * weight streaming follow encode_forward (dit.c:2577-3038): resident blocks run
 * from device memory; the rest are copied from pinned host memory into two
 * alternating device slots on the copy stream, the copy for block b+1 overlapping
 * the compute of block b. The modulation comes from the 256-d sinusoidal
 * timestep features of dit_schedule.c:152-162 (cos for the first half, sin for
 * the second) through a small time MLP, computed once at creation as the
 * reference precomputes its per-step modulation. */
#include "h3_dit_synth.h"
#include "h3_gpu_surface.h"
#include "h3_safetensors.h"
#include "h3_hip_ext.h"
#include "h3_quant.h"
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define SLOTS 6u
#define TIME_FEATURES 256u
#define PROJ 4 /* qkv, out, up, down */

/* Stages of one block kept when config.trace_block selects it, in op order. */
enum { T_X0, T_XN1, T_QKV, T_Q, T_K, T_V, T_ATTN, T_O, T_X1, T_XN2, T_H, T_ACT, T_F, T_X2, TRACE_COUNT };
static const char *const TRACE_NAMES[TRACE_COUNT] = {"x0", "xn1", "qkv", "q", "k", "v", "attn", "o", "x1",
                                                     "xn2", "h", "act", "f", "x2"};

struct h3_hip_dit_synth {
    h3_gpu *gpu;
    h3_hip_dit_synth_config c;
    uint32_t video_rows, rows;
    /* weights */
    h3_gpu_tensor **proj;          /* [blocks][PROJ], NULL for streamed blocks */
    h3_gpu_tensor *slot[2][PROJ];  /* streaming slots */
    void **host;                   /* [blocks] pinned copies of streamed blocks */
    size_t host_bytes[PROJ];
    h3_gpu_tensor **norm1, **norm2, **mod; /* per block */
    h3_gpu_tensor *patch, *head, *head_norm, *head_mod;
    /* activations and tables */
    h3_gpu_tensor **qn, **kn;      /* per block Q/K RMSNorm weights [128] (qk_norm) */
    h3_gpu_tensor *latent, *latent_bf16, *x, *xn, *qkv, *q, *k, *v, *attn, *o, *h, *act, *f, *vel;
    h3_sol_block *layout_blocks;   /* attention_mode 4: the bound 64-row layout */
    h3_gpu_tensor *cos_t, *sin_t, *row_map;
    uint64_t kept, total;
    h3_gpu_tensor *trace[TRACE_COUNT]; /* copies of the traced block's stages */
    /* With trace_block set: the modulation chain's inputs and intermediates
     * (time features, both time projections, SiLU input, shared projection,
     * the traced block's own table), kept for the parity tests. */
    h3_gpu_tensor *mod_trace[6];
};
static const char *const MOD_TRACE_NAMES[6] = {"time.features", "time.w1", "time.w2", "time.t1", "time.shared",
                                               "trace.mod_table"};

static int fail(char *error, size_t size, const char *fmt, ...) {
    if (error && size) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(error, size, fmt, ap);
        va_end(ap);
    }
    return 0;
}

h3_hip_dit_synth_config h3_hip_dit_synth_default(void) {
    h3_hip_dit_synth_config c;
    memset(&c, 0, sizeof(c));
    c.blocks = 40; c.hidden = 5120; c.heads = 40; c.mlp = 13824;
    c.frames = 27; c.height = 30; c.width = 40; c.audio_rows = 1024;
    c.latent = 256; c.streamed_first = 20; c.mask_density = 0.25f;
    c.attention_mode = 1; c.eps = 1e-6f; c.time = 0.5f; c.seed = 5;
    c.rope_half = 64; c.subblock_sparsity = 0.75f;
    return c;
}

h3_hip_dit_synth_config h3_hip_dit_synth_h3(void) {
    h3_hip_dit_synth_config c = h3_hip_dit_synth_default();
    c.blocks = 50; c.hidden = 5376; c.heads = 56; c.mlp = 14336;
    c.frames = 25; c.height = 27; c.width = 27; c.audio_rows = 0;
    c.streamed_first = 50; c.mask_density = -1.f; c.attention_mode = 0; c.eps = 1e-5f;
    c.rope_half = 48; c.swiglu = 1; c.qk_norm = 1; c.grouped_qkv = 1;
    return c;
}

static uint16_t to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* BF16 tensor of `n` values offset + spread * N(0,1) from the device generator. */
static h3_gpu_tensor *normal_tensor(h3_gpu *g, size_t n, uint64_t seed, float spread, float offset) {
    h3_gpu_tensor *t = h3_gpu_tensor_new_bf16(g, n);
    if (!t) return NULL;
    if (!h3_hip_fill_normal_bf16(g, t, seed, spread, n)) { h3_gpu_tensor_free(t); return NULL; }
    if (offset != 0.f) {
        uint16_t *host = malloc(n * 2);
        if (!host) { h3_gpu_tensor_free(t); return NULL; }
        if (!h3_gpu_synchronize(g) || !h3_gpu_tensor_read_bf16(t, host, n)) { free(host); h3_gpu_tensor_free(t); return NULL; }
        for (size_t i = 0; i < n; i++) {
            uint32_t u = (uint32_t)host[i] << 16;
            float v;
            memcpy(&v, &u, 4);
            host[i] = to_bf16(v + offset);
        }
        int ok = h3_gpu_tensor_write_bf16(t, host, n);
        free(host);
        if (!ok) { h3_gpu_tensor_free(t); return NULL; }
    }
    return t;
}

int h3_hip_dit_rope_tables(uint32_t frames, uint32_t height, uint32_t width, uint32_t audio_rows, uint32_t half,
                           uint16_t *cosines, uint16_t *sines) {
    if (!frames || !height || !width || !cosines || !sines || (half != 64 && (!half || half > 64 || half % 3)))
        return 0;
    /* Pairs per axis (frame, row, column): 22/21/21 for half 64 (44/42/42
     * channels), else half / 3 each. */
    uint32_t split[3] = {22, 21, 21};
    if (half != 64) split[0] = split[1] = split[2] = half / 3;
    float inv[64];
    for (uint32_t axis = 0, j = 0; axis < 3; axis++)
        for (uint32_t i = 0; i < split[axis]; i++, j++)
            inv[j] = (float)pow(10000.0, -2.0 * (double)i / (2.0 * split[axis]));
    const uint32_t video = frames * height * width;
    for (uint32_t r = 0; r < video + audio_rows; r++) {
        float pos[3] = {0.f, 0.f, 0.f};
        if (r < video) {
            pos[0] = (float)(r / (height * width));
            pos[1] = (float)((r / width) % height);
            pos[2] = (float)(r % width);
        }
        for (uint32_t axis = 0, j = 0; axis < 3; axis++)
            for (uint32_t i = 0; i < split[axis]; i++, j++) {
                float angle = pos[axis] * inv[j];
                cosines[(size_t)r * half + j] = to_bf16(cosf(angle));
                sines[(size_t)r * half + j] = to_bf16(sinf(angle));
            }
    }
    return 1;
}

void h3_hip_dit_time_features(const float *times, uint32_t rows, float *features) {
    for (uint32_t row = 0; row < rows; row++)
        for (uint32_t i = 0; i < TIME_FEATURES / 2; i++) {
            float freq = expf(-logf(10000.0f) * (float)i / (float)(TIME_FEATURES / 2));
            float angle = times[row] * freq;
            features[(size_t)row * TIME_FEATURES + i] = cosf(angle);
            features[(size_t)row * TIME_FEATURES + TIME_FEATURES / 2 + i] = sinf(angle);
        }
}

/* 3D RoPE tables over the video grid; audio rows get angle 0. */
static int rope_tables(h3_hip_dit_synth *m) {
    const uint32_t half = m->c.rope_half;
    size_t n = (size_t)m->rows * half;
    uint16_t *c = malloc(n * 2), *s = malloc(n * 2);
    int ok = c && s && h3_hip_dit_rope_tables(m->c.frames, m->c.height, m->c.width, m->c.audio_rows, half, c, s);
    if (ok) {
        m->cos_t = h3_gpu_tensor_from_bf16(m->gpu, c, n);
        m->sin_t = h3_gpu_tensor_from_bf16(m->gpu, s, n);
    }
    free(c); free(s);
    return ok && m->cos_t && m->sin_t;
}

/* Modulation [2 rows (video, audio), 6 slots, hidden] per block = a shared time
 * projection of the timestep features plus a per-block table; the head uses 2
 * slots (shift, scale). */
static int modulation(h3_hip_dit_synth *m, char *error, size_t size) {
    h3_gpu *g = m->gpu;
    const uint32_t H = m->c.hidden;
    float feat[2 * TIME_FEATURES], times[2] = {m->c.time, m->c.time};
    uint16_t featb[2 * TIME_FEATURES];
    h3_hip_dit_time_features(times, 2, feat);
    for (uint32_t i = 0; i < 2 * TIME_FEATURES; i++) featb[i] = to_bf16(feat[i]);
    uint64_t sd = m->c.seed * 1000003ull;
    h3_gpu_tensor *tf = h3_gpu_tensor_from_bf16(g, featb, 2 * TIME_FEATURES);
    h3_gpu_tensor *w1 = normal_tensor(g, (size_t)H * TIME_FEATURES, sd + 1, 1.0f / 16.0f, 0.f);
    h3_gpu_tensor *w2 = normal_tensor(g, (size_t)SLOTS * H * H, sd + 2, 0.1f / sqrtf((float)H), 0.f);
    h3_gpu_tensor *t1 = h3_gpu_tensor_new_bf16(g, 2 * (size_t)H), *t2 = h3_gpu_tensor_new_bf16(g, 2 * (size_t)H);
    h3_gpu_tensor *shared = h3_gpu_tensor_new_bf16(g, 2 * (size_t)SLOTS * H);
    int ok = tf && w1 && w2 && t1 && t2 && shared &&
             h3_gpu_linear_bf16(g, t1, tf, w1, NULL, 2, TIME_FEATURES, H) &&
             h3_gpu_silu_bf16(g, t2, t1, 2 * H) &&
             h3_gpu_linear_bf16(g, shared, t2, w2, NULL, 2, H, SLOTS * H);
    for (uint32_t b = 0; ok && b < m->c.blocks; b++) {
        h3_gpu_tensor *table = normal_tensor(g, 2 * (size_t)SLOTS * H, sd + 100 + b, 0.05f, 0.f);
        m->mod[b] = h3_gpu_tensor_new_bf16(g, 2 * (size_t)SLOTS * H);
        ok = table && m->mod[b] && h3_gpu_add_bf16(g, m->mod[b], shared, table, 2 * SLOTS * H) && h3_gpu_synchronize(g);
        if (ok && m->c.trace_block == b + 1) m->mod_trace[5] = table;
        else h3_gpu_tensor_free(table);
    }
    m->head_mod = ok ? normal_tensor(g, 2 * 2 * (size_t)H, sd + 3, 0.05f, 0.f) : NULL;
    ok = ok && m->head_mod && h3_gpu_synchronize(g);
    if (ok && m->c.trace_block) {
        m->mod_trace[0] = tf; m->mod_trace[1] = w1; m->mod_trace[2] = w2;
        m->mod_trace[3] = t1; m->mod_trace[4] = shared;
        tf = w1 = w2 = t1 = shared = NULL;
    }
    h3_gpu_tensor_free(tf); h3_gpu_tensor_free(w1); h3_gpu_tensor_free(w2);
    h3_gpu_tensor_free(t1); h3_gpu_tensor_free(t2); h3_gpu_tensor_free(shared);
    return ok ? 1 : fail(error, size, "modulation: %s", h3_gpu_error(g));
}

static void proj_shape(const h3_hip_dit_synth_config *c, int j, uint32_t *n, uint32_t *k) {
    const uint32_t inner = c->heads * 128;
    switch (j) {
    case 0: *n = 3 * inner; *k = c->hidden; break;
    case 1: *n = c->hidden; *k = inner; break;
    case 2: *n = c->swiglu ? 2 * c->mlp : c->mlp; *k = c->hidden; break;
    default: *n = c->hidden; *k = c->mlp; break;
    }
}

static h3_gpu_tensor *q8_random(h3_gpu *g, uint32_t n, uint32_t k, uint64_t seed) {
    h3_gpu_tensor *t = h3_hip_q8_new(g, n, k, k);
    if (t && !h3_hip_fill_q8_random(g, t, seed, 1e-3f, 1e-2f)) { h3_gpu_tensor_free(t); t = NULL; }
    return t;
}

/* Quantized projection weight (projection_quant 1 FP8, 2 NVFP4): N(0, 1/k)
 * BF16 values packed to the mode's descriptor. */
static h3_gpu_tensor *quant_random(h3_gpu *g, uint32_t n, uint32_t k, uint64_t seed) {
    h3_gpu_tensor *b = normal_tensor(g, (size_t)n * k, seed, 1.0f / sqrtf((float)k), 0.f);
    if (!b) return NULL;
    h3_gpu_tensor *t = h3_gpu_synchronize(g) ? h3_hip_quant_weight_from_bf16(g, b, n, k) : NULL;
    h3_gpu_tensor_free(b);
    return t;
}

static int weights(h3_hip_dit_synth *m, char *error, size_t size) {
    h3_gpu *g = m->gpu;
    const h3_hip_dit_synth_config *c = &m->c;
    uint32_t streamed = c->blocks - (c->streamed_first < c->blocks ? c->streamed_first : c->blocks);
    for (int j = 0; j < PROJ; j++) {
        uint32_t n, k;
        proj_shape(c, j, &n, &k);
        m->host_bytes[j] = (size_t)n * k + (size_t)n * 4;
        if (streamed)
            for (int s = 0; s < 2; s++)
                if (!(m->slot[s][j] = h3_hip_q8_new(g, n, k, k))) return fail(error, size, "slot: %s", h3_gpu_error(g));
    }
    size_t block_bytes = 0;
    for (int j = 0; j < PROJ; j++) block_bytes += m->host_bytes[j];
    for (uint32_t b = 0; b < c->blocks; b++) {
        int resident = b < c->streamed_first;
        if (!resident && !(m->host[b] = h3_hip_host_alloc(g, block_bytes)))
            return fail(error, size, "pinned block %u: %s", b, h3_gpu_error(g));
        size_t at = 0;
        for (int j = 0; j < PROJ; j++) {
            uint32_t n, k;
            proj_shape(c, j, &n, &k);
            h3_gpu_tensor *t = c->projection_quant ? quant_random(g, n, k, c->seed * 7919ull + b * 8 + j)
                                                   : q8_random(g, n, k, c->seed * 7919ull + b * 8 + j);
            if (!t) return fail(error, size, "block %u weight %d: %s", b, j, h3_gpu_error(g));
            if (resident) m->proj[(size_t)b * PROJ + j] = t;
            else {
                int ok = h3_gpu_synchronize(g) && h3_hip_tensor_copy_to_host(t, (char *)m->host[b] + at, m->host_bytes[j]);
                h3_gpu_tensor_free(t);
                if (!ok) return fail(error, size, "block %u host copy: %s", b, h3_gpu_error(g));
            }
            at += m->host_bytes[j];
        }
        m->norm1[b] = normal_tensor(g, c->hidden, c->seed * 31 + 2 * b, 0.1f, 1.0f);
        m->norm2[b] = normal_tensor(g, c->hidden, c->seed * 31 + 2 * b + 1, 0.1f, 1.0f);
        if (c->qk_norm) {
            m->qn[b] = normal_tensor(g, 128, c->seed * 43 + 2 * b, 0.1f, 1.0f);
            m->kn[b] = normal_tensor(g, 128, c->seed * 43 + 2 * b + 1, 0.1f, 1.0f);
            if (!m->qn[b] || !m->kn[b]) return fail(error, size, "qk norms: %s", h3_gpu_error(g));
        }
        if (!m->norm1[b] || !m->norm2[b] || !h3_gpu_synchronize(g)) return fail(error, size, "norms: %s", h3_gpu_error(g));
    }
    m->patch = normal_tensor(g, (size_t)c->hidden * c->latent, c->seed * 37 + 1, 1.0f / sqrtf((float)c->latent), 0.f);
    m->head = normal_tensor(g, (size_t)c->latent * c->hidden, c->seed * 37 + 2, 1.0f / sqrtf((float)c->hidden), 0.f);
    m->head_norm = normal_tensor(g, c->hidden, c->seed * 37 + 3, 0.1f, 1.0f);
    if (!m->patch || !m->head || !m->head_norm || !h3_gpu_synchronize(g)) return fail(error, size, "head: %s", h3_gpu_error(g));
    return 1;
}

static h3_gpu_tensor *bf16_buffer(h3_gpu *g, size_t n) { return h3_gpu_tensor_new_bf16(g, n); }

h3_hip_dit_synth *h3_hip_dit_synth_create(h3_gpu *g, const h3_hip_dit_synth_config *config, char *error, size_t size) {
    if (!g || !config) { fail(error, size, "missing context or config"); return NULL; }
    const h3_hip_dit_synth_config *c = config;
    if (!c->blocks || !c->heads || !c->mlp || c->mlp % 256 || !c->hidden || c->hidden % 256 || !c->latent ||
        c->latent % 256 || !c->frames || !c->height || !c->width ||
        (c->rope_half != 64 && (!c->rope_half || c->rope_half > 64 || c->rope_half % 3)) ||
        (c->attention_mode != 0 && c->attention_mode != 1 && c->attention_mode != 4) ||
        (c->projection_quant < 0 || c->projection_quant > 2) || c->trace_block > c->blocks) {
        fail(error, size, "synthetic DiT: hidden/mlp/latent multiples of 256, rope_half 64 or a multiple of 3 "
                          "below it, attention mode 0/1/4, projection_quant 0/1/2, trace_block <= blocks");
        return NULL;
    }
    if (c->projection_quant && c->streamed_first < c->blocks) {
        fail(error, size, "synthetic DiT: quantized projections need every block resident");
        return NULL;
    }
    h3_hip_dit_synth *m = calloc(1, sizeof(*m));
    if (!m) { fail(error, size, "out of host memory"); return NULL; }
    m->gpu = g;
    m->c = *c;
    m->video_rows = c->frames * c->height * c->width;
    m->rows = m->video_rows + c->audio_rows;
    m->proj = calloc((size_t)c->blocks * PROJ, sizeof(*m->proj));
    m->host = calloc(c->blocks, sizeof(*m->host));
    m->norm1 = calloc(c->blocks, sizeof(*m->norm1));
    m->norm2 = calloc(c->blocks, sizeof(*m->norm2));
    m->mod = calloc(c->blocks, sizeof(*m->mod));
    m->qn = calloc(c->blocks, sizeof(*m->qn));
    m->kn = calloc(c->blocks, sizeof(*m->kn));
    if (!m->proj || !m->host || !m->norm1 || !m->norm2 || !m->mod || !m->qn || !m->kn) {
        fail(error, size, "out of host memory");
        goto bad;
    }
    if (!h3_gpu_dit_attention_configure(g, c->attention_mode)) {
        fail(error, size, "attention configure: %s", h3_gpu_error(g));
        goto bad;
    }
    if (c->projection_quant) {
        /* Synthetic weights are packed in place; checkpoints go through the
         * artifact cache. No H3 admission bytes: every block is resident. */
        const char *tmp = getenv("TMPDIR");
        char cache[512];
        snprintf(cache, sizeof(cache), "%s/h3cli-amd-quant", tmp && *tmp ? tmp : "/tmp");
        if (!h3_gpu_quant_configure(g, c->projection_quant, cache, 0, 0, 0)) {
            fail(error, size, "quant configure: %s", h3_gpu_error(g));
            goto bad;
        }
    }
    if (!h3_gpu_begin(g)) { fail(error, size, "begin: %s", h3_gpu_error(g)); goto bad; }
    if (!weights(m, error, size) || !modulation(m, error, size) || !rope_tables(m)) { h3_gpu_cancel(g); goto bad; }
    {
        const size_t R = m->rows, H = c->hidden, I = (size_t)c->heads * 128;
        uint32_t *map = malloc(R * 4);
        if (!map) { h3_gpu_cancel(g); goto bad; }
        for (size_t r = 0; r < R; r++) map[r] = r < m->video_rows ? 0u : 1u;
        m->row_map = h3_gpu_tensor_from_u32(g, map, R);
        free(map);
        m->latent = h3_gpu_tensor_new_f32(g, R * c->latent);
        m->latent_bf16 = bf16_buffer(g, R * c->latent);
        m->x = bf16_buffer(g, R * H); m->xn = bf16_buffer(g, R * H);
        m->qkv = bf16_buffer(g, R * I * 3);
        m->q = bf16_buffer(g, R * I); m->k = bf16_buffer(g, R * I); m->v = bf16_buffer(g, R * I);
        m->attn = bf16_buffer(g, R * I); m->o = bf16_buffer(g, R * H);
        m->h = bf16_buffer(g, R * c->mlp * (c->swiglu ? 2 : 1)); m->f = bf16_buffer(g, R * H);
        m->act = c->swiglu || c->projection_quant ? bf16_buffer(g, R * c->mlp) : NULL;
        m->vel = bf16_buffer(g, R * c->latent);
        if (!m->row_map || !m->latent || !m->latent_bf16 || !m->x || !m->xn || !m->qkv || !m->q || !m->k || !m->v ||
            !m->attn || !m->o || !m->h || !m->f || !m->vel || ((c->swiglu || c->projection_quant) && !m->act)) {
            fail(error, size, "activations: %s", h3_gpu_error(g));
            h3_gpu_cancel(g);
            goto bad;
        }
        if (c->trace_block) {
            const size_t sizes[TRACE_COUNT] = {R * H, R * H, R * I * 3, R * I, R * I, R * I, R * I, R * H, R * H,
                                               R * H, R * c->mlp * (c->swiglu ? 2 : 1), m->act ? R * c->mlp : 0,
                                               R * H, R * H};
            for (int i = 0; i < TRACE_COUNT; i++)
                if (sizes[i] && !(m->trace[i] = bf16_buffer(g, sizes[i]))) {
                    fail(error, size, "trace: %s", h3_gpu_error(g));
                    h3_gpu_cancel(g);
                    goto bad;
                }
        }
        /* Seeded N(0,1) latent. */
        h3_gpu_tensor *init = normal_tensor(g, R * c->latent, c->seed * 41 + 1, 1.0f, 0.f);
        int ok = init && h3_gpu_cast_bf16_to_f32(g, m->latent, init, (uint32_t)(R * c->latent)) && h3_gpu_synchronize(g);
        h3_gpu_tensor_free(init);
        if (!ok) { fail(error, size, "latent: %s", h3_gpu_error(g)); h3_gpu_cancel(g); goto bad; }
    }
    if (!h3_gpu_submit(g)) { fail(error, size, "setup: %s", h3_gpu_error(g)); goto bad; }
    if (c->attention_mode == 4) {
        /* SubBlock: the router runs over a 64-row layout with no protected
         * blocks, at the request's sparsity, from the first step (warmup off). */
        uint32_t nb = (m->rows + 63) / 64;
        m->layout_blocks = calloc(nb, sizeof(*m->layout_blocks));
        if (!m->layout_blocks) goto bad;
        for (uint32_t b = 0; b < nb; b++) m->layout_blocks[b].rows = m->rows - b * 64 < 64 ? m->rows - b * 64 : 64;
        h3_sol_layout layout = {m->rows, nb, nb, 0, m->layout_blocks, m->layout_blocks};
        if (!h3_hip_dit_subblock_policy(g, c->subblock_sparsity, -1) || !h3_gpu_dit_sol_layout(g, &layout)) {
            fail(error, size, "subblock layout: %s", h3_gpu_error(g));
            goto bad;
        }
        m->kept = m->total = (uint64_t)nb * nb;
    } else if (c->mask_density >= 0.f) {
        uint32_t blocks = (m->rows + 127) / 128;
        uint8_t *mask = malloc((size_t)blocks * blocks);
        if (!mask) goto bad;
        m->kept = h3_hip_synthetic_block_mask(mask, m->rows, m->video_rows, 128, c->mask_density, c->seed);
        m->total = (uint64_t)blocks * blocks;
        int ok = m->kept && h3_hip_dit_block_mask(g, mask, blocks, blocks, 128);
        free(mask);
        if (!ok) { fail(error, size, "mask: %s", h3_gpu_error(g)); goto bad; }
    } else {
        uint32_t blocks = (m->rows + 127) / 128;
        m->kept = m->total = (uint64_t)blocks * blocks;
    }
    return m;
bad:
    h3_hip_dit_synth_free(m);
    return NULL;
}

void h3_hip_dit_synth_free(h3_hip_dit_synth *m) {
    if (!m) return;
    h3_gpu *g = m->gpu;
    if (m->proj) for (size_t i = 0; i < (size_t)m->c.blocks * PROJ; i++) h3_gpu_tensor_free(m->proj[i]);
    for (int s = 0; s < 2; s++) for (int j = 0; j < PROJ; j++) h3_gpu_tensor_free(m->slot[s][j]);
    size_t block_bytes = 0;
    for (int j = 0; j < PROJ; j++) block_bytes += m->host_bytes[j];
    if (m->host) for (uint32_t b = 0; b < m->c.blocks; b++) h3_hip_host_free(g, m->host[b], block_bytes);
    for (uint32_t b = 0; b < m->c.blocks; b++) {
        if (m->norm1) h3_gpu_tensor_free(m->norm1[b]);
        if (m->norm2) h3_gpu_tensor_free(m->norm2[b]);
        if (m->mod) h3_gpu_tensor_free(m->mod[b]);
        if (m->qn) h3_gpu_tensor_free(m->qn[b]);
        if (m->kn) h3_gpu_tensor_free(m->kn[b]);
    }
    h3_gpu_tensor *all[] = {m->patch, m->head, m->head_norm, m->head_mod, m->latent, m->latent_bf16, m->x, m->xn,
                            m->qkv, m->q, m->k, m->v, m->attn, m->o, m->h, m->act, m->f, m->vel, m->cos_t, m->sin_t,
                            m->row_map};
    for (size_t i = 0; i < sizeof(all) / sizeof(*all); i++) h3_gpu_tensor_free(all[i]);
    for (int i = 0; i < TRACE_COUNT; i++) h3_gpu_tensor_free(m->trace[i]);
    for (int i = 0; i < 6; i++) h3_gpu_tensor_free(m->mod_trace[i]);
    free(m->proj); free(m->host); free(m->norm1); free(m->norm2); free(m->mod); free(m->qn); free(m->kn);
    free(m->layout_blocks);
    free(m);
}

/* Device copy of a stage of the traced block into its trace tensor. */
static int keep(h3_hip_dit_synth *m, int stage, const h3_gpu_tensor *src) {
    h3_gpu_tensor *t = m->trace[stage];
    return !t || h3_gpu_copy_bf16(m->gpu, t, 0, src, 0, h3_gpu_tensor_elements(t));
}

/* Queue the copy of streamed block b into its slot (b % 2) on the copy stream. */
static int prefetch(h3_hip_dit_synth *m, uint32_t b) {
    if (b >= m->c.blocks || b < m->c.streamed_first) return 1;
    size_t at = 0;
    for (int j = 0; j < PROJ; j++) {
        if (!h3_hip_tensor_stream_host(m->slot[b % 2][j], (const char *)m->host[b] + at, m->host_bytes[j])) return 0;
        at += m->host_bytes[j];
    }
    return 1;
}

int h3_hip_dit_synth_step(h3_hip_dit_synth *m, int step, float dt) {
    if (!m) return 0;
    h3_gpu *g = m->gpu;
    const h3_hip_dit_synth_config *c = &m->c;
    const uint32_t R = m->rows, H = c->hidden, L = c->latent, I = c->heads * 128;
    const float scale = 1.0f / sqrtf(128.0f);
    if (!h3_gpu_begin(g)) return 0;
    int ok = h3_gpu_dit_attention_noise(g, step, 0.5f, 0.5f) && prefetch(m, c->streamed_first) &&
             h3_gpu_cast_f32_to_bf16(g, m->latent_bf16, m->latent, R * L) &&
             h3_gpu_linear_bf16(g, m->x, m->latent_bf16, m->patch, NULL, R, L, H);
    for (uint32_t b = 0; ok && b < c->blocks; b++) {
        h3_gpu_tensor **w = b < c->streamed_first ? &m->proj[(size_t)b * PROJ] : m->slot[b % 2];
        /* The next streamed block's copy overlaps this block's compute. */
        if (b + 1 > c->streamed_first && !prefetch(m, b + 1)) { ok = 0; break; }
        const h3_gpu_tensor *qn = c->qk_norm ? m->qn[b] : NULL, *kn = c->qk_norm ? m->kn[b] : NULL;
        const int tr = c->trace_block == b + 1;
        ok = (!tr || keep(m, T_X0, m->x)) &&
             h3_gpu_adaln_bf16(g, m->xn, m->x, m->norm1[b], m->mod[b], m->row_map, R, H, SLOTS, 0, 1, c->eps);
        if (c->grouped_qkv)
            ok = ok && h3_gpu_grouped_qkv_linear_rope_bf16(g, m->q, m->k, m->v, m->qkv, m->xn, w[0], qn, kn, m->cos_t,
                                                           m->sin_t, R, H, c->heads, 128, c->rope_half, c->eps);
        else
            ok = ok && h3_gpu_linear_bf16(g, m->qkv, m->xn, w[0], NULL, R, H, 3 * I) &&
                 h3_gpu_qkv_rope_bf16(g, m->q, m->k, m->v, m->qkv, qn, kn, m->cos_t, m->sin_t, R, c->heads, 128,
                                      c->rope_half, c->eps);
        ok = ok && (!tr || (keep(m, T_XN1, m->xn) && keep(m, T_QKV, m->qkv) && keep(m, T_Q, m->q) &&
                            keep(m, T_K, m->k) && keep(m, T_V, m->v)));
        ok = ok && h3_gpu_dit_sdpa_bf16(g, m->attn, m->q, m->k, m->v, R, c->heads, 128, scale, 0, b, step) &&
             h3_gpu_linear_bf16(g, m->o, m->attn, w[1], NULL, R, I, H) &&
             (!tr || (keep(m, T_ATTN, m->attn) && keep(m, T_O, m->o))) &&
             h3_gpu_gate_adaln_bf16(g, m->x, m->xn, m->x, m->o, m->norm2[b], m->mod[b], m->mod[b], m->row_map, R, H,
                                    SLOTS, 2, 3, 4, c->eps) &&
             (!tr || (keep(m, T_X1, m->x) && keep(m, T_XN2, m->xn)));
        if (c->swiglu) {
            ok = ok && h3_gpu_linear_bf16(g, m->h, m->xn, w[2], NULL, R, H, 2 * c->mlp) &&
                 h3_gpu_swiglu_bf16(g, m->act, m->h, R, c->mlp) &&
                 h3_gpu_linear_bf16(g, m->f, m->act, w[3], NULL, R, c->mlp, H);
        } else if (c->projection_quant) {
            /* Packed weights take no epilogue: GELU-tanh separately. */
            ok = ok && h3_gpu_linear_bf16(g, m->h, m->xn, w[2], NULL, R, H, c->mlp) &&
                 h3_gpu_gelu_bf16(g, m->act, m->h, (uint32_t)(R * c->mlp), 1) &&
                 h3_gpu_linear_bf16(g, m->f, m->act, w[3], NULL, R, c->mlp, H);
        } else {
            ok = ok && h3_hip_linear_gelu_bf16(g, m->h, m->xn, w[2], NULL, R, H, c->mlp) &&
                 h3_gpu_linear_bf16(g, m->f, m->h, w[3], NULL, R, c->mlp, H);
        }
        ok = ok && (!tr || (keep(m, T_H, m->h) && (!m->act || keep(m, T_ACT, m->act)) && keep(m, T_F, m->f))) &&
             h3_gpu_gate_bf16(g, m->x, m->x, m->f, m->mod[b], m->row_map, R, H, SLOTS, 5) &&
             (!tr || keep(m, T_X2, m->x));
    }
    ok = ok && h3_gpu_adaln_bf16(g, m->xn, m->x, m->head_norm, m->head_mod, m->row_map, R, H, 2, 0, 1, c->eps) &&
         h3_gpu_linear_bf16(g, m->vel, m->xn, m->head, NULL, R, H, L) &&
         h3_gpu_euler_bf16(g, m->latent, 0, m->vel, m->vel, R * L, dt, 0.0f);
    if (!ok) {
        h3_gpu_cancel(g);
        return 0;
    }
    return h3_gpu_submit(g);
}

/* Checkpoint names of a block's tensors (dit.c:604-611) in load order; the
 * projections map to PROJ slots 0-3. */
static const char *const BLOCK_NAMES[8] = {"attn.qkv_proj.weight", "attn.out_proj.weight", "mlp.fc1.weight",
                                           "mlp.fc2.weight", "norm1.weight", "norm2.weight",
                                           "attn.q_norm.weight", "attn.k_norm.weight"};

static h3_gpu_tensor **block_slot(h3_hip_dit_synth *m, uint32_t b, int i) {
    switch (i) {
    case 4: return &m->norm1[b];
    case 5: return &m->norm2[b];
    case 6: return &m->qn[b];
    case 7: return &m->kn[b];
    default: return b < m->c.streamed_first ? &m->proj[(size_t)b * PROJ + i] : NULL;
    }
}

/* Expected [rows, columns] of tensor i (columns 0 for a vector). */
static void block_shape(const h3_hip_dit_synth_config *c, int i, uint32_t *rows, uint32_t *cols) {
    if (i < PROJ) { proj_shape(c, i, rows, cols); return; }
    *rows = i < 6 ? c->hidden : 128;
    *cols = 0;
}

int h3_hip_dit_synth_load(h3_hip_dit_synth *m, const char *path, char *error, size_t size) {
    if (!m || !path) return fail(error, size, "missing model or path");
    const h3_hip_dit_synth_config *c = &m->c;
    if (c->streamed_first < c->blocks) return fail(error, size, "checkpoint loading needs every block resident");
    h3_st_header header;
    if (!h3_st_read_header(path, &header, error, size)) return 0;
    h3_gpu *g = m->gpu;
    int ok = 1;
    char name[160];
    /* Validate everything before replacing anything. */
    for (uint32_t b = 0; ok && b < c->blocks; b++)
        for (int i = 0; ok && i < 8; i++) {
            if (i >= 6 && !c->qk_norm) continue;
            uint32_t rows, cols;
            block_shape(c, i, &rows, &cols);
            snprintf(name, sizeof(name), "blocks.%u.%s", b, BLOCK_NAMES[i]);
            const h3_st_tensor *t = h3_st_find(&header, name);
            int shape_ok = t && t->dtype == H3_DTYPE_BF16 &&
                           (cols ? t->ndim == 2 && t->shape[0] == rows && t->shape[1] == cols
                                 : t->ndim == 1 && t->shape[0] == rows);
            if (!shape_ok) ok = fail(error, size, "missing/invalid %s", name);
        }
    for (uint32_t b = 0; ok && b < c->blocks; b++)
        for (int i = 0; ok && i < 8; i++) {
            if (i >= 6 && !c->qk_norm) continue;
            uint32_t rows, cols;
            block_shape(c, i, &rows, &cols);
            snprintf(name, sizeof(name), "blocks.%u.%s", b, BLOCK_NAMES[i]);
            const h3_st_tensor *t = h3_st_find(&header, name);
            h3_gpu_tensor *loaded = !cols ? h3_gpu_tensor_load_bf16(g, path, t->file_offset, rows)
                                    : c->projection_quant ? h3_gpu_quant_load(g, path, t->file_offset, rows, cols)
                                                          : h3_gpu_q8_load(g, path, t->file_offset, rows, cols);
            if (!loaded) { ok = fail(error, size, "%s: %s", name, h3_gpu_error(g)); break; }
            h3_gpu_tensor **slot = block_slot(m, b, i);
            h3_gpu_tensor_free(*slot);
            *slot = loaded;
        }
    h3_st_free_header(&header);
    return ok;
}

h3_gpu_tensor *h3_hip_dit_synth_tensor(h3_hip_dit_synth *m, const char *name) {
    if (!m || !name) return NULL;
    if (!strcmp(name, "latent")) return m->latent;
    if (!strcmp(name, "hidden")) return m->x;
    if (!strcmp(name, "velocity")) return m->vel;
    if (!strcmp(name, "latent_bf16")) return m->latent_bf16;
    if (!strcmp(name, "patch")) return m->patch;
    if (!strcmp(name, "head")) return m->head;
    if (!strcmp(name, "head_norm")) return m->head_norm;
    if (!strcmp(name, "head_mod")) return m->head_mod;
    if (!strcmp(name, "rope_cos")) return m->cos_t;
    if (!strcmp(name, "rope_sin")) return m->sin_t;
    if (!strcmp(name, "row_map")) return m->row_map;
    for (int i = 0; i < 6; i++)
        if (!strcmp(name, MOD_TRACE_NAMES[i])) return m->mod_trace[i];
    if (!strncmp(name, "trace.", 6)) {
        for (int i = 0; i < TRACE_COUNT; i++)
            if (!strcmp(name + 6, TRACE_NAMES[i])) return m->trace[i];
        return NULL;
    }
    unsigned b, used = 0;
    if (sscanf(name, "blocks.%u.%n", &b, &used) != 1 || !used || b >= m->c.blocks) return NULL;
    if (!strcmp(name + used, "modulation")) return m->mod[b];
    for (int i = 0; i < 8; i++)
        if (!strcmp(name + used, BLOCK_NAMES[i])) {
            h3_gpu_tensor **slot = block_slot(m, b, i);
            return slot ? *slot : NULL;
        }
    return NULL;
}

uint32_t h3_hip_dit_synth_rows(const h3_hip_dit_synth *m) { return m ? m->rows : 0; }

uint64_t h3_hip_dit_synth_kept_blocks(const h3_hip_dit_synth *m, uint64_t *total) {
    if (total) *total = m ? m->total : 0;
    return m ? m->kept : 0;
}
