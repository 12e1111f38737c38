/*
 * pa_oracle.c -- CPU oracle for the paged-attention path. TEST INFRASTRUCTURE ONLY: loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker / CPU baseline,
 * never by the product library. See pa_oracle.h for the contract of each function.
 *
 * Reference paths are relative to the werwedc/ml-framework root; PA = src/MLFramework/Inference/
 * PagedAttention, Q = src/MLFramework/Quantization/Operations.
 */
#include "pa_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------------ */
/* bf16: src/MLFramework/Amp/BFloat16.cs:99-107 (ConvertToBFloat16: bits >> 16) and :109-117
 * (ConvertToFloat: bits << 16). */
uint16_t orc_bf16_from_f32(float v) {
    uint32_t bits;
    memcpy(&bits, &v, 4);
    return (uint16_t)(bits >> 16);
}

float orc_f32_from_bf16(uint16_t b) {
    uint32_t bits = ((uint32_t)b) << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* ------------------------------------------------------------------------------------------ */
/* Q/QuantizationUtils.cs:146-159:
 *   NaN -> 0; +/-Inf -> int.MaxValue / int.MinValue;
 *   (int)Math.CopySign(Math.Floor(Math.Abs(value) + 0.5f), value)
 * Math.Abs(float) and the + 0.5f are fp32 operations; Floor/CopySign run on the double the fp32
 * sum widens to; the double -> int cast saturates (.NET 9 conversion semantics). */
int32_t orc_round_half_away_from_zero(float v) {
    if (isnan(v)) return 0;
    if (isinf(v)) return v > 0 ? INT32_MAX : INT32_MIN;
    volatile float a = fabsf(v) + 0.5f; /* fp32 add, kept in fp32 */
    double r = copysign(floor((double)a), (double)v);
    if (r >= 2147483647.0) return INT32_MAX;
    if (r <= -2147483648.0) return INT32_MIN;
    return (int32_t)r;
}

/* Q/QuantizationUtils.cs:110-115 (Clamp(int,int,int)). */
static int32_t orc_clamp_i(int32_t v, int32_t lo, int32_t hi) {
    if (v < lo) return lo;
    if (v > hi) return hi;
    return v;
}

/* Q/QuantizationOperations.cs:188-200: NaN -> (quantMin + quantMax) / 2 = (-128 + 127) / 2 = 0
 * (C# integer division truncates); otherwise clamp(RoundHalfAwayFromZero(value / scale)). */
int8_t orc_quantize_symmetric(float v, float scale) {
    if (isnan(v)) return (int8_t)((-128 + 127) / 2);
    volatile float scaled = v / scale; /* IEEE fp32 division */
    int32_t r = orc_round_half_away_from_zero(scaled);
    return (int8_t)orc_clamp_i(r, -128, 127);
}

/* Q/QuantizationOperations.cs:83-88: (q - zeroPoint) * scale in fp32, zero point 0. */
float orc_dequantize(int8_t q, float scale) {
    volatile float r = (float)((int32_t)q - 0) * scale;
    return r;
}

/* ------------------------------------------------------------------------------------------ */
/* PA/Kernels/StandardPagedAttentionKernel.cs:270-278 (GetTensorValue, row-major 4-D index). */
static inline float orc_get(const float* t, int s1, int s2, int s3, int b, int q, int h, int d) {
    return t[(size_t)b * ((size_t)s1 * s2 * s3) + (size_t)q * ((size_t)s2 * s3) + (size_t)h * s3 + d];
}

/* PA/Kernels/StandardPagedAttentionKernel.cs:21-84 and the helpers it calls. */
int orc_sdpa(const float* q, const float* k, const float* v, float* out,
             int batch, int nq, int nc, int H, int D, int phase, float scale, int force_causal) {
    if (!q || !k || !v || !out || batch < 0 || nq < 0 || nc < 0 || H <= 0 || D <= 0) return -1;
    if (batch == 0 || nq == 0) return 0;
    /* :18 and :28 -- default scale 1/MathF.Sqrt(headDim), overridden only when scale > 0. */
    const float default_scale = 1.0f / sqrtf((float)D);
    const float actual = scale > 0 ? scale : default_scale;

    const size_t n_scores = (size_t)batch * nq * H * (size_t)nc;
    float* scores = (float*)malloc((n_scores ? n_scores : 1) * sizeof(float));
    float* weights = (float*)malloc((n_scores ? n_scores : 1) * sizeof(float));
    if (!scores || !weights) { free(scores); free(weights); return -1; }

    /* MatmulQueryKey, :86-129 -- loops b, h, q, c, d; sum += qVal * kVal (unfused). */
    for (int b = 0; b < batch; b++)
        for (int h = 0; h < H; h++)
            for (int qi = 0; qi < nq; qi++)
                for (int c = 0; c < nc; c++) {
                    float sum = 0.0f;
                    for (int d = 0; d < D; d++) {
                        float qv = orc_get(q, nq, H, D, b, qi, h, d);
                        float kv = orc_get(k, nc, H, D, b, c, h, d);
                        sum += qv * kv;
                    }
                    size_t idx = (size_t)b * ((size_t)nq * H * nc) + (size_t)qi * ((size_t)H * nc) +
                                 (size_t)h * nc + c;
                    scores[idx] = sum;
                }

    /* ScaleTensor, :257-268 -- applied after the dot product. */
    for (size_t i = 0; i < n_scores; i++) scores[i] = scores[i] * actual;

    /* ApplyCausalMask, :57-66 (condition) and :219-255 (bottom-right aligned:
     * startPos = numCached - numQueries; keys c > startPos + q are -inf). */
    if ((phase == PA_PHASE_DECODE && nc > nq) || force_causal) {
        int start = nc - nq;
        for (int b = 0; b < batch; b++)
            for (int h = 0; h < H; h++)
                for (int qi = 0; qi < nq; qi++)
                    for (int c = start + qi + 1; c < nc; c++) {
                        if (c < 0) continue;
                        size_t idx = (size_t)b * ((size_t)nq * H * nc) + (size_t)qi * ((size_t)H * nc) +
                                     (size_t)h * nc + c;
                        scores[idx] = -INFINITY;
                    }
    }

    /* Softmax, :175-217 -- max (init -inf, strict >), MathF.Exp(x - max), sequential sum,
     * then each term divided by the sum. */
    const size_t outer = (size_t)batch * nq * H;
    for (size_t i = 0; i < outer; i++) {
        float mx = -INFINITY;
        for (int j = 0; j < nc; j++)
            if (scores[i * nc + j] > mx) mx = scores[i * nc + j];
        float sum = 0.0f;
        for (int j = 0; j < nc; j++) {
            weights[i * nc + j] = expf(scores[i * nc + j] - mx);
            sum += weights[i * nc + j];
        }
        for (int j = 0; j < nc; j++) weights[i * nc + j] /= sum;
    }

    /* MatmulWeightValue, :131-173 -- loops b, h, q, d, c; sum += wVal * vVal (unfused). */
    for (int b = 0; b < batch; b++)
        for (int h = 0; h < H; h++)
            for (int qi = 0; qi < nq; qi++)
                for (int d = 0; d < D; d++) {
                    float sum = 0.0f;
                    for (int c = 0; c < nc; c++) {
                        size_t widx = (size_t)b * ((size_t)nq * H * nc) + (size_t)qi * ((size_t)H * nc) +
                                      (size_t)h * nc + c;
                        float wv = weights[widx];
                        float vv = orc_get(v, nc, H, D, b, c, h, d);
                        sum += wv * vv;
                    }
                    out[(size_t)b * ((size_t)nq * H * D) + (size_t)qi * ((size_t)H * D) + (size_t)h * D + d] = sum;
                }

    free(scores);
    free(weights);
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* PA/KVCacheBlockManager.cs -- a FIFO ring standing in for ConcurrentQueue<int>. */
struct orc_block_manager {
    int32_t* ring;
    int32_t cap, head, count;
};

orc_block_manager* orc_bm_create(int32_t total_blocks) {
    if (total_blocks < 0) return NULL;
    orc_block_manager* bm = (orc_block_manager*)calloc(1, sizeof(*bm));
    if (!bm) return NULL;
    bm->cap = total_blocks > 0 ? total_blocks : 1;
    bm->ring = (int32_t*)malloc(sizeof(int32_t) * (size_t)bm->cap);
    if (!bm->ring) { free(bm); return NULL; }
    /* :59-62 -- for (i = 0; i < totalBlocks; i++) Enqueue(i). */
    for (int32_t i = 0; i < total_blocks; i++) bm->ring[i] = i;
    bm->count = total_blocks;
    return bm;
}

void orc_bm_destroy(orc_block_manager* bm) {
    if (!bm) return;
    free(bm->ring);
    free(bm);
}

/* :70-75 -- TryDequeue, else Failed("No free blocks available") (-1 here). */
int32_t orc_bm_allocate_block(orc_block_manager* bm) {
    if (!bm || bm->count == 0) return -1;
    int32_t id = bm->ring[bm->head];
    bm->head = (bm->head + 1) % bm->cap;
    bm->count--;
    return id;
}

/* :157-174 -- Enqueue at the tail. Ids that were never handed out are ignored, as FreeBlock
 * ignores ids missing from _blocks. */
void orc_bm_free_block(orc_block_manager* bm, int32_t block_id) {
    if (!bm || block_id < 0 || block_id >= bm->cap || bm->count >= bm->cap) return;
    bm->ring[(bm->head + bm->count) % bm->cap] = block_id;
    bm->count++;
}

/* :120-152 -- allocate one by one; on failure free the ones taken (to the tail) and return an
 * empty list. */
int32_t orc_bm_allocate_blocks(orc_block_manager* bm, int32_t count, int32_t* out) {
    if (!bm || count < 0 || (count > 0 && !out)) return 0;
    for (int32_t i = 0; i < count; i++) {
        int32_t id = orc_bm_allocate_block(bm);
        if (id < 0) {
            for (int32_t j = 0; j < i; j++) orc_bm_free_block(bm, out[j]);
            return 0;
        }
        out[i] = id;
    }
    return count;
}

int32_t orc_bm_free_count(const orc_block_manager* bm) { return bm ? bm->count : 0; }

/* ------------------------------------------------------------------------------------------ */
void orc_build_slot_mapping(const pa_config* cfg, const int32_t* block_tables,
                            int32_t max_blocks_per_seq, const int32_t* start_pos,
                            const int32_t* num_new, const int32_t* token_offset, int32_t num_seqs,
                            int64_t* slot_mapping) {
    const int32_t B = cfg->block_size;
    for (int32_t s = 0; s < num_seqs; s++) {
        for (int32_t j = 0; j < num_new[s]; j++) {
            int64_t p = (int64_t)start_pos[s] + j;
            int64_t logical = p / B;
            int64_t slot = -1;
            if (p >= 0 && logical < max_blocks_per_seq) {
                int32_t blk = block_tables[(size_t)s * max_blocks_per_seq + logical];
                if (blk >= 0) slot = (int64_t)blk * B + p % B;
            }
            slot_mapping[token_offset[s] + j] = slot;
        }
    }
}

/* ------------------------------------------------------------------------------------------ */
static float orc_load_act(const void* p, int32_t dtype, size_t i) {
    if (dtype == PA_DTYPE_BF16) return orc_f32_from_bf16(((const uint16_t*)p)[i]);
    return ((const float*)p)[i];
}

static int orc_slot_valid(const pa_config* cfg, int64_t slot) {
    return slot >= 0 && slot < (int64_t)cfg->num_blocks * cfg->block_size;
}

/* Element (row `off` of block `blk`, KV head h, dim d) in the cache layout of pa_config:
 * K tiles are row-major [block_size][head_dim], V tiles are dim-major [head_dim][block_size]. */
static size_t orc_cache_index(const pa_config* cfg, int is_v, int64_t blk, int32_t h, int64_t off, int32_t d) {
    const size_t tile = ((size_t)blk * cfg->num_kv_heads + h) * (size_t)cfg->block_size * cfg->head_dim;
    return is_v ? tile + (size_t)d * cfg->block_size + off : tile + (size_t)off * cfg->head_dim + d;
}

/* One cache (K or V) of one append call. */
static void orc_append_one(const pa_config* cfg, int is_v, const void* x_new, const int64_t* sm,
                           int32_t n_tok, void* cache, float* scale, float* absmax) {
    const int32_t B = cfg->block_size, H = cfg->num_kv_heads, D = cfg->head_dim;
    if (cfg->kv_dtype != PA_DTYPE_INT8) {
        for (int32_t i = 0; i < n_tok; i++) {
            if (!orc_slot_valid(cfg, sm[i])) continue;
            int64_t blk = sm[i] / B, off = sm[i] % B;
            for (int32_t h = 0; h < H; h++)
                for (int32_t d = 0; d < D; d++) {
                    float x = orc_load_act(x_new, cfg->q_dtype, ((size_t)i * H + h) * D + d);
                    size_t o = orc_cache_index(cfg, is_v, blk, h, off, d);
                    if (cfg->kv_dtype == PA_DTYPE_BF16) ((uint16_t*)cache)[o] = orc_bf16_from_f32(x);
                    else ((float*)cache)[o] = x;
                }
        }
        return;
    }
    /* int8: segments = maximal runs of consecutive valid tokens that land in one block. */
    int8_t* c8 = (int8_t*)cache;
    int32_t i = 0;
    while (i < n_tok) {
        if (!orc_slot_valid(cfg, sm[i])) { i++; continue; }
        int64_t blk = sm[i] / B;
        int32_t j = i + 1;
        while (j < n_tok && orc_slot_valid(cfg, sm[j]) && sm[j] / B == blk) j++;
        /* slots written by this segment, and whether it starts the block (offset 0) */
        uint64_t written = 0;
        int fresh = 0;
        for (int32_t t = i; t < j; t++) {
            int64_t off = sm[t] % B;
            written |= (uint64_t)1 << off;
            if (off == 0) fresh = 1;
        }
        for (int32_t h = 0; h < H; h++) {
            float seg_amax = 0.0f;
            for (int32_t t = i; t < j; t++)
                for (int32_t d = 0; d < D; d++) {
                    float a = fabsf(orc_load_act(x_new, cfg->q_dtype, ((size_t)t * H + h) * D + d));
                    if (a > seg_amax) seg_amax = a;
                }
            size_t sidx = (size_t)blk * H + h;
            float old_amax = fresh ? 0.0f : absmax[sidx];
            float old_scale = fresh ? 0.0f : scale[sidx];
            float cur_scale = old_scale;
            if (fresh) {
                absmax[sidx] = seg_amax;
                cur_scale = seg_amax / 127.0f;
                scale[sidx] = cur_scale;
            } else if (seg_amax > old_amax) {
                volatile float ns = seg_amax / 127.0f;
                cur_scale = ns;
                for (int32_t off = 0; off < B; off++) {
                    if (written & ((uint64_t)1 << off)) continue;
                    for (int32_t d = 0; d < D; d++) {
                        size_t o = orc_cache_index(cfg, is_v, blk, h, off, d);
                        c8[o] = orc_quantize_symmetric(orc_dequantize(c8[o], old_scale), cur_scale);
                    }
                }
                absmax[sidx] = seg_amax;
                scale[sidx] = cur_scale;
            }
            for (int32_t t = i; t < j; t++) {
                int64_t off = sm[t] % B;
                for (int32_t d = 0; d < D; d++) {
                    float x = orc_load_act(x_new, cfg->q_dtype, ((size_t)t * H + h) * D + d);
                    c8[orc_cache_index(cfg, is_v, blk, h, off, d)] = orc_quantize_symmetric(x, cur_scale);
                }
            }
        }
        i = j;
    }
}

int orc_kv_append(const pa_config* cfg, const void* k_new, const void* v_new,
                  const int64_t* slot_mapping, int32_t n_tok, void* k_cache, void* v_cache,
                  float* k_scale, float* v_scale, float* k_absmax, float* v_absmax) {
    if (!cfg || n_tok < 0) return -1;
    if (n_tok == 0) return 0;
    if (!k_new || !v_new || !slot_mapping || !k_cache || !v_cache) return -1;
    if (cfg->block_size <= 0 || cfg->block_size > 64) return -1;
    if (cfg->kv_dtype == PA_DTYPE_INT8 && (!k_scale || !v_scale || !k_absmax || !v_absmax)) return -1;
    orc_append_one(cfg, 0, k_new, slot_mapping, n_tok, k_cache, k_scale, k_absmax);
    orc_append_one(cfg, 1, v_new, slot_mapping, n_tok, v_cache, v_scale, v_absmax);
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* Gather of the first T tokens of one sequence into the dense [1][T][Hq][D] fp32 layout the
 * reference kernel takes -- the intended PagedAttentionLayer.GatherKVFromBlocks /
 * DecodeOrchestrator.GatherDecodeKeys (Layers/PagedAttentionLayer.cs:368-389,
 * Phases/DecodeOrchestrator.cs:111-123): token t lives at block table[t / B], row t % B.
 * KV head h / G feeds query head h (GQA by head repetition). Tokens in an invalid block read 0. */
static void orc_gather(const pa_config* cfg, int is_v, const void* cache, const float* scales,
                       const int32_t* table, int32_t max_blocks, int32_t T, float* dst) {
    const int32_t B = cfg->block_size, Hkv = cfg->num_kv_heads, Hq = cfg->num_q_heads, D = cfg->head_dim;
    const int32_t G = Hq / Hkv;
    for (int32_t t = 0; t < T; t++) {
        int32_t lb = t / B;
        int32_t blk = lb < max_blocks ? table[lb] : -1;
        int valid = blk >= 0 && blk < cfg->num_blocks;
        for (int32_t h = 0; h < Hq; h++) {
            int32_t kh = h / G;
            float* row = dst + ((size_t)t * Hq + h) * D;
            if (!valid) { memset(row, 0, sizeof(float) * (size_t)D); continue; }
            for (int32_t d = 0; d < D; d++) {
                size_t o = orc_cache_index(cfg, is_v, blk, kh, t % B, d);
                float x;
                if (cfg->kv_dtype == PA_DTYPE_BF16) x = orc_f32_from_bf16(((const uint16_t*)cache)[o]);
                else if (cfg->kv_dtype == PA_DTYPE_INT8)
                    x = orc_dequantize(((const int8_t*)cache)[o], scales[(size_t)blk * Hkv + kh]);
                else x = ((const float*)cache)[o];
                row[d] = x;
            }
        }
    }
}

static int orc_cfg_ok(const pa_config* cfg) {
    return cfg && cfg->block_size > 0 && cfg->num_q_heads > 0 && cfg->num_kv_heads > 0 &&
           cfg->head_dim > 0 && cfg->num_q_heads % cfg->num_kv_heads == 0 && cfg->num_blocks >= 0 &&
           (cfg->kv_dtype == PA_DTYPE_FP32 || cfg->kv_dtype == PA_DTYPE_BF16 || cfg->kv_dtype == PA_DTYPE_INT8) &&
           (cfg->q_dtype == PA_DTYPE_FP32 || cfg->q_dtype == PA_DTYPE_BF16);
}

int orc_paged_decode(const pa_config* cfg, float* out, const void* q,
                     const void* k_cache, const void* v_cache,
                     const float* k_scale, const float* v_scale,
                     const int32_t* block_tables, const int32_t* context_lens,
                     int32_t num_seqs, int32_t max_blocks_per_seq, int32_t n_threads) {
    if (!orc_cfg_ok(cfg) || num_seqs < 0 || max_blocks_per_seq < 0) return -1;
    if (num_seqs == 0) return 0;
    if (!out || !q || !k_cache || !v_cache || !block_tables || !context_lens) return -1;
    if (cfg->kv_dtype == PA_DTYPE_INT8 && (!k_scale || !v_scale)) return -1;
    const int32_t Hq = cfg->num_q_heads, D = cfg->head_dim;
    int err = 0;
#ifdef _OPENMP
    if (n_threads < 1) n_threads = 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(n_threads) reduction(| : err)
#else
    (void)n_threads;
#endif
    for (int32_t s = 0; s < num_seqs; s++) {
        int32_t T = context_lens[s];
        if (T > max_blocks_per_seq * cfg->block_size) T = max_blocks_per_seq * cfg->block_size;
        float* o = out + (size_t)s * Hq * D;
        if (T <= 0) { memset(o, 0, sizeof(float) * (size_t)Hq * D); continue; }
        float* qs = (float*)malloc(sizeof(float) * (size_t)Hq * D);
        float* ks = (float*)malloc(sizeof(float) * (size_t)T * Hq * D);
        float* vs = (float*)malloc(sizeof(float) * (size_t)T * Hq * D);
        if (!qs || !ks || !vs) { free(qs); free(ks); free(vs); err |= 1; continue; }
        for (int32_t i = 0; i < Hq * D; i++) qs[i] = orc_load_act(q, cfg->q_dtype, (size_t)s * Hq * D + i);
        const int32_t* table = block_tables + (size_t)s * max_blocks_per_seq;
        orc_gather(cfg, 0, k_cache, k_scale, table, max_blocks_per_seq, T, ks);
        orc_gather(cfg, 1, v_cache, v_scale, table, max_blocks_per_seq, T, vs);
        err |= orc_sdpa(qs, ks, vs, o, 1, 1, T, Hq, D, PA_PHASE_DECODE, cfg->scale, 0) != 0;
        free(qs); free(ks); free(vs);
    }
    return err ? -1 : 0;
}

int orc_chunked_prefill(const pa_config* cfg, float* out, const void* q,
                        const int32_t* q_start_loc, const int32_t* prefix_lens,
                        const void* k_cache, const void* v_cache,
                        const float* k_scale, const float* v_scale,
                        const int32_t* block_tables, int32_t num_seqs,
                        int32_t max_blocks_per_seq, int32_t n_threads) {
    if (!orc_cfg_ok(cfg) || num_seqs < 0 || max_blocks_per_seq < 0) return -1;
    if (num_seqs == 0) return 0;
    if (!out || !q || !q_start_loc || !prefix_lens || !k_cache || !v_cache || !block_tables) return -1;
    if (cfg->kv_dtype == PA_DTYPE_INT8 && (!k_scale || !v_scale)) return -1;
    const int32_t Hq = cfg->num_q_heads, D = cfg->head_dim;
    const int literal = (cfg->flags & PA_FLAG_REFERENCE_LITERAL_MASK) != 0;
    const int no_mask = (cfg->flags & PA_FLAG_NO_MASK) != 0;
    int err = 0;
    if (n_threads < 1) n_threads = 1;
    /* Sequences one after another; the heads of a sequence are independent problems (the
     * reference loops over them inside one call, :29-49), so they run in parallel. */
    for (int32_t s = 0; s < num_seqs; s++) {
        int32_t L = q_start_loc[s + 1] - q_start_loc[s];
        int32_t P = prefix_lens[s];
        int32_t T = P + L;
        if (L <= 0) continue;
        float* o = out + (size_t)q_start_loc[s] * Hq * D;
        if (P < 0 || T > max_blocks_per_seq * cfg->block_size) { err |= 1; continue; }
        float* ks = (float*)malloc(sizeof(float) * (size_t)T * Hq * D);
        float* vs = (float*)malloc(sizeof(float) * (size_t)T * Hq * D);
        if (!ks || !vs) { free(ks); free(vs); err |= 1; continue; }
        const int32_t* table = block_tables + (size_t)s * max_blocks_per_seq;
        orc_gather(cfg, 0, k_cache, k_scale, table, max_blocks_per_seq, T, ks);
        orc_gather(cfg, 1, v_cache, v_scale, table, max_blocks_per_seq, T, vs);
        const int phase = no_mask ? PA_PHASE_PREFILL : PA_PHASE_DECODE;
        const int force = (!no_mask && !literal) ? 1 : 0;
        const size_t q_base = (size_t)q_start_loc[s] * Hq * D;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(n_threads) reduction(| : err)
#else
        (void)n_threads;
#endif
        for (int32_t h = 0; h < Hq; h++) {
            float* qh = (float*)malloc(sizeof(float) * (size_t)L * D);
            float* kh = (float*)malloc(sizeof(float) * (size_t)T * D);
            float* vh = (float*)malloc(sizeof(float) * (size_t)T * D);
            float* oh = (float*)malloc(sizeof(float) * (size_t)L * D);
            if (!qh || !kh || !vh || !oh) { free(qh); free(kh); free(vh); free(oh); err |= 1; continue; }
            for (int32_t i = 0; i < L; i++)
                for (int32_t d = 0; d < D; d++)
                    qh[(size_t)i * D + d] = orc_load_act(q, cfg->q_dtype, q_base + ((size_t)i * Hq + h) * D + d);
            for (int32_t t = 0; t < T; t++) {
                memcpy(kh + (size_t)t * D, ks + ((size_t)t * Hq + h) * D, sizeof(float) * (size_t)D);
                memcpy(vh + (size_t)t * D, vs + ((size_t)t * Hq + h) * D, sizeof(float) * (size_t)D);
            }
            err |= orc_sdpa(qh, kh, vh, oh, 1, L, T, 1, D, phase, cfg->scale, force) != 0;
            for (int32_t i = 0; i < L; i++)
                memcpy(o + ((size_t)i * Hq + h) * D, oh + (size_t)i * D, sizeof(float) * (size_t)D);
            free(qh); free(kh); free(vh); free(oh);
        }
        free(ks); free(vs);
    }
    return err ? -1 : 0;
}
