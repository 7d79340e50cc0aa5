/*
 * CPU restatement of simpler's paged-attention decode — TEST INFRASTRUCTURE ONLY.
 *
 * Used by tests/ (as a second, independent restatement next to pa_oracle.py)
 * and by bench.py's cpu_baseline leg (timed, kind "port"). Nothing in the
 * product library links or calls it.
 *
 * The per-block work restates the four AICore kernels the reference submits
 * for every KV block (examples/a2a3/tensormap_and_ringbuffer/paged_attention/
 * kernels/):
 *   qk_block()      <- aic/aic_qk_matmul.cpp:38-100      sij = qi * kj^T (fp32 acc of bf16)
 *   softmax_block() <- aiv/aiv_softmax_prepare.cpp:96-131 pad -inf, *scale, rowmax,
 *                                                        exp, bf16 round (p), rowsum of
 *                                                        the rounded p
 *                      (fully masked rows: m = -1e30, l = 0, p = 0 as in
 *                       tests/st/.../batch_paged_attention/kernels/aiv/
 *                       aiv_softmax_prepare.cpp:105-121 and goldens/paged_attention.py:160)
 *   pv_block()      <- aic/aic_pv_matmul.cpp:38-99       oi_new = pij * vj
 *   online_update() <- aiv/aiv_online_update.cpp:125-224 first-block copy, merge
 *                                                        (m', alpha, beta, l', o'),
 *                                                        last-block divide
 * driven per (batch, kv head) the way the orchestration walks blocks
 * (kernels/orchestration/paged_attention_orch.cpp:163-249), generalised to
 * GQA rows (kv_head = h / group), a causal multi-token query and MLA
 * (V = the first Dv columns of K).
 *
 * Threads: pthreads over (batch, kv head) work items; n_threads <= 0 uses 1.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    const uint16_t *q, *k, *v;
    const int32_t *block_table, *context_lens;
    float *out;
    int batch, q_len, num_heads, kv_heads, dk, dv, block_size, max_blocks;
    float scale;
    int causal, mla;
    /* work distribution */
    int n_items;
    int next_item;
    pthread_mutex_t mu;
} OracleJob;

static inline float bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline float round_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return x; /* NaN */
    u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
    float r;
    memcpy(&r, &u, 4);
    return r;
}

/* One (batch, kv_head) item: rows r = i*g + hh for query token i and group head hh. */
static void run_item(const OracleJob *j, int item, float *scratch) {
    const int b = item / j->kv_heads, kvh = item % j->kv_heads;
    const int g = j->num_heads / j->kv_heads;
    const int rows = j->q_len * g;
    const int bs = j->block_size, dk = j->dk, dv = j->dv;
    const int ctx = j->context_lens[b];
    const int nblk = (ctx + bs - 1) / bs;
    const size_t krow = (size_t)j->kv_heads * dk;            /* token stride in K */
    const size_t vrow = (size_t)j->kv_heads * (j->mla ? dk : dv);
    const uint16_t *vsrc = j->mla ? j->k : j->v;

    float *qf = scratch;                     /* rows*dk */
    float *sij = qf + (size_t)rows * dk;     /* rows*bs */
    float *oi_new = sij + (size_t)rows * bs; /* rows*dv */
    float *oi = oi_new + (size_t)rows * dv;  /* rows*dv */
    float *mi = oi + (size_t)rows * dv;      /* rows */
    float *li = mi + rows;
    float *mij = li + rows;
    float *lij = mij + rows;
    int *rlen = (int *)(lij + rows);

    for (int r = 0; r < rows; r++) {
        const int i = r / g, hh = r % g;
        const uint16_t *src = j->q + (((size_t)b * j->q_len + i) * j->num_heads + (size_t)kvh * g + hh) * dk;
        for (int d = 0; d < dk; d++) qf[(size_t)r * dk + d] = bf16_to_f32(src[d]);
        rlen[r] = j->causal ? ctx - (j->q_len - 1 - i) : ctx;
    }

    for (int bn = 0; bn < nblk; bn++) {
        const int blk = j->block_table[(size_t)b * j->max_blocks + bn];
        const uint16_t *kb = j->k + ((size_t)blk * bs * j->kv_heads + kvh) * dk;
        const uint16_t *vb = vsrc + ((size_t)blk * bs * j->kv_heads + kvh) * (j->mla ? dk : dv);

        /* QK: sij[r][t] = sum_d q[r][d] * k[t][d] */
        for (int r = 0; r < rows; r++) {
            const float *qr = qf + (size_t)r * dk;
            for (int t = 0; t < bs; t++) {
                const uint16_t *kt = kb + (size_t)t * krow;
                float acc = 0.f;
                for (int d = 0; d < dk; d++) acc += qr[d] * bf16_to_f32(kt[d]);
                sij[(size_t)r * bs + t] = acc;
            }
        }
        /* softmax prepare: mask, scale, rowmax, exp, bf16 round, rowsum */
        for (int r = 0; r < rows; r++) {
            int valid = rlen[r] - bn * bs;
            if (valid > bs) valid = bs;
            if (valid < 0) valid = 0;
            float *s = sij + (size_t)r * bs;
            float m = -INFINITY;
            for (int t = 0; t < bs; t++) {
                s[t] = (t < valid) ? s[t] * j->scale : -INFINITY;
                if (s[t] > m) m = s[t];
            }
            if (m < -1e30f) m = -1e30f;
            float l = 0.f;
            for (int t = 0; t < bs; t++) {
                const float p = (t < valid) ? round_bf16(expf(s[t] - m)) : 0.f;
                s[t] = p;
                l += p;
            }
            mij[r] = m;
            lij[r] = l;
        }
        /* PV: oi_new[r][d] = sum_t p[r][t] * v[t][d] */
        for (int r = 0; r < rows; r++) {
            float *o = oi_new + (size_t)r * dv;
            for (int d = 0; d < dv; d++) o[d] = 0.f;
            const float *p = sij + (size_t)r * bs;
            for (int t = 0; t < bs; t++) {
                if (p[t] == 0.f) continue;
                const uint16_t *vt = vb + (size_t)t * vrow;
                for (int d = 0; d < dv; d++) o[d] += p[t] * bf16_to_f32(vt[d]);
            }
        }
        /* online update */
        if (bn == 0) {
            memcpy(mi, mij, sizeof(float) * rows);
            memcpy(li, lij, sizeof(float) * rows);
            memcpy(oi, oi_new, sizeof(float) * (size_t)rows * dv);
        } else {
            for (int r = 0; r < rows; r++) {
                const float mn = mi[r] > mij[r] ? mi[r] : mij[r];
                const float alpha = expf(mi[r] - mn), beta = expf(mij[r] - mn);
                li[r] = alpha * li[r] + beta * lij[r];
                float *o = oi + (size_t)r * dv;
                const float *on = oi_new + (size_t)r * dv;
                for (int d = 0; d < dv; d++) o[d] = alpha * o[d] + beta * on[d];
                mi[r] = mn;
            }
        }
    }
    for (int r = 0; r < rows; r++) {
        const int i = r / g, hh = r % g;
        float *dst = j->out + (((size_t)b * j->q_len + i) * j->num_heads + (size_t)kvh * g + hh) * dv;
        for (int d = 0; d < dv; d++) dst[d] = (nblk > 0 && li[r] > 0.f) ? oi[(size_t)r * dv + d] / li[r] : 0.f;
    }
}

static size_t scratch_floats(const OracleJob *j) {
    const int g = j->num_heads / j->kv_heads;
    const size_t rows = (size_t)j->q_len * g;
    return rows * j->dk + rows * j->block_size + 2 * rows * j->dv + 5 * rows + 16;
}

static void *worker(void *arg) {
    OracleJob *j = (OracleJob *)arg;
    float *scratch = (float *)malloc(sizeof(float) * scratch_floats(j));
    if (!scratch) return NULL;
    for (;;) {
        pthread_mutex_lock(&j->mu);
        const int item = j->next_item++;
        pthread_mutex_unlock(&j->mu);
        if (item >= j->n_items) break;
        run_item(j, item, scratch);
    }
    free(scratch);
    return NULL;
}

/*
 * Full decode over all (batch, kv head) items, or over the first `n_items`
 * of them when 0 < n_items < batch*kv_heads (bounded CPU-baseline sample).
 * q: bf16 [B, q_len, Hq, Dk]; k: bf16 [nblk, BS, Hkv, Dk]; v: bf16 [nblk, BS, Hkv, Dv]
 * (ignored when mla != 0: V = K[..., :Dv]); out: fp32 [B, q_len, Hq, Dv].
 * Returns 0, or -1 on invalid arguments.
 */
int pa_oracle_decode(const uint16_t *q, const uint16_t *k, const uint16_t *v, const int32_t *block_table,
                     const int32_t *context_lens, float *out, int batch, int q_len, int num_heads, int kv_heads,
                     int dk, int dv, int block_size, int max_blocks, float scale, int causal, int mla,
                     int n_threads, int n_items) {
    if (batch < 0 || q_len < 1 || kv_heads < 1 || num_heads % kv_heads || dk < 1 || dv < 1 || block_size < 1)
        return -1;
    if (mla && dv > dk) return -1;
    OracleJob j;
    memset(&j, 0, sizeof(j));
    j.q = q; j.k = k; j.v = v; j.block_table = block_table; j.context_lens = context_lens; j.out = out;
    j.batch = batch; j.q_len = q_len; j.num_heads = num_heads; j.kv_heads = kv_heads; j.dk = dk; j.dv = dv;
    j.block_size = block_size; j.max_blocks = max_blocks; j.scale = scale; j.causal = causal; j.mla = mla;
    const int total = batch * kv_heads;
    j.n_items = (n_items > 0 && n_items < total) ? n_items : total;
    pthread_mutex_init(&j.mu, NULL);
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 256) n_threads = 256;
    pthread_t th[256];
    for (int t = 0; t < n_threads; t++) pthread_create(&th[t], NULL, worker, &j);
    for (int t = 0; t < n_threads; t++) pthread_join(th[t], NULL);
    pthread_mutex_destroy(&j.mu);
    return 0;
}
