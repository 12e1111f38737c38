/*
 * pa_oracle.h -- CPU oracle for the paged-attention path. TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the reference's CPU algorithm (werwedc/ml-framework, C#) and
 * of the paging / int8 policies the build fixes on top of it. Only tests/, __graft_entry__.smoke()
 * and the cpu_baseline leg of bench.py may load it, and only as the checker (or the timed CPU
 * baseline) -- never as the product path. The product (libpa_hip.so) does not link it.
 *
 * Every function cites the reference file:line it follows (paths relative to the reference
 * root). How each function is pinned (golden vectors, known-answer tests, closed forms,
 * brute force) is listed in tests/test_oracle.py; functions without such a check are marked
 * "parity unpinned" here. None is currently unpinned.
 *
 * Built with -O2 -ffp-contract=off and without -ffast-math so that `sum += a * b` stays an
 * unfused fp32 multiply followed by an fp32 add, as RyuJIT's scalar code evaluates it.
 */
#ifndef PA_ORACLE_H
#define PA_ORACLE_H

#include <stdint.h>
#include "../include/paged_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* bf16 <-> fp32, src/MLFramework/Amp/BFloat16.cs:99-117 (truncation, no rounding). */
uint16_t orc_bf16_from_f32(float v);
float orc_f32_from_bf16(uint16_t b);

/* QuantizationUtils.RoundHalfAwayFromZero, src/MLFramework/Quantization/Operations/
 * QuantizationUtils.cs:146-159, with .NET 9's saturating double->int conversion. */
int32_t orc_round_half_away_from_zero(float v);
/* QuantizationOperations.QuantizeSymmetric (int8 range), QuantizationOperations.cs:188-200. */
int8_t orc_quantize_symmetric(float v, float scale);
/* QuantizationOperations.Dequantize with zero point 0, QuantizationOperations.cs:83-88. */
float orc_dequantize(int8_t q, float scale);

/* StandardPagedAttentionKernel.ComputePagedAttention,
 * src/MLFramework/Inference/PagedAttention/Kernels/StandardPagedAttentionKernel.cs:21-84.
 * q: [batch][nq][H][D], k, v: [batch][nc][H][D], out: [batch][nq][H][D], all fp32.
 * phase: PA_PHASE_PREFILL / PA_PHASE_DECODE. scale <= 0 selects 1/sqrtf(D) (:18, :28).
 * force_causal != 0 applies the bottom-right causal mask even where the reference's condition
 * (phase == Decode && nc > nq, :57) is false. Returns 0, or -1 on bad arguments. */
int orc_sdpa(const float* q, const float* k, const float* v, float* out,
             int batch, int nq, int nc, int H, int D, int phase, float scale, int force_causal);

/* KVCacheBlockManager free list, src/MLFramework/Inference/PagedAttention/
 * KVCacheBlockManager.cs:59-62 (ids 0..N-1 queued in order), :70-112 (AllocateBlock dequeues the
 * head; -1 = "No free blocks available"), :120-152 (AllocateBlocks all-or-nothing with rollback
 * that re-enqueues at the tail), :157-174 (FreeBlock enqueues at the tail). */
typedef struct orc_block_manager orc_block_manager;
orc_block_manager* orc_bm_create(int32_t total_blocks);
void orc_bm_destroy(orc_block_manager* bm);
int32_t orc_bm_allocate_block(orc_block_manager* bm);
/* Writes `count` ids to out and returns count, or returns 0 and allocates nothing. */
int32_t orc_bm_allocate_blocks(orc_block_manager* bm, int32_t count, int32_t* out);
void orc_bm_free_block(orc_block_manager* bm, int32_t block_id);
int32_t orc_bm_free_count(const orc_block_manager* bm);

/* Slot mapping, the closed form of the intended BlockTable mapping
 * (tests/MLFramework.Tests/Inference/PagedAttention/BlockTableTests.cs:115-134: block k of a
 * sequence holds tokens [k*B, (k+1)*B)) and PagedAttentionLayer.UpdateKVCache's position in
 * block (Layers/PagedAttentionLayer.cs:256-272). Same contract as pa_build_slot_mapping. */
void orc_build_slot_mapping(const pa_config* cfg, const int32_t* block_tables,
                            int32_t max_blocks_per_seq, const int32_t* start_pos,
                            const int32_t* num_new, const int32_t* token_offset, int32_t num_seqs,
                            int64_t* slot_mapping);

/* KV append with the cache layout and int8 policy of pa_kv_append (include/paged_attn.h).
 * k_new/v_new are cfg->q_dtype (FP32 floats or BF16 uint16). Element quantisation is
 * orc_quantize_symmetric; requantisation of resident codes is
 * QuantizeSymmetric(Dequantize(q, old_scale), new_scale). Returns 0 or -1. */
int orc_kv_append(const pa_config* cfg, const void* k_new, const void* v_new,
                  const int64_t* slot_mapping, int32_t n_tok, void* k_cache, void* v_cache,
                  float* k_scale, float* v_scale, float* k_absmax, float* v_absmax);

/* Ragged paged decode: for each sequence, gather its first context_lens[s] tokens through its
 * block table (dequantised to fp32), repeat each KV head for its Hq/Hkv query heads and call
 * orc_sdpa with batch 1, one query and phase Decode -- DecodeOrchestrator.BatchDecode /
 * ComputeDecodeAttention (Phases/DecodeOrchestrator.cs:64-109), one call per sequence.
 * A sequence with context_len <= 0 yields zeros. n_threads > 1 runs sequences in parallel
 * (OpenMP); results do not depend on it. Returns 0 or -1. */
int orc_paged_decode(const pa_config* cfg, float* out, const void* q,
                     const void* k_cache, const void* v_cache,
                     const float* k_scale, const float* v_scale,
                     const int32_t* block_tables, const int32_t* context_lens,
                     int32_t num_seqs, int32_t max_blocks_per_seq, int32_t n_threads);

/* Chunked prefill: for each sequence, its chunk's queries (positions prefix .. prefix+L-1) attend
 * to keys [0, prefix+L) gathered like orc_paged_decode; orc_sdpa with phase Decode and
 * force_causal unless cfg->flags has PA_FLAG_REFERENCE_LITERAL_MASK (then the reference's own
 * condition decides); PA_FLAG_NO_MASK calls it with phase Prefill (never masked). */
int orc_chunked_prefill(const pa_config* cfg, float* out, const void* q,
                        const int32_t* q_start_loc, const int32_t* prefix_lens,
                        const void* k_cache, const void* v_cache,
                        const float* k_scale, const float* v_scale,
                        const int32_t* block_tables, int32_t num_seqs,
                        int32_t max_blocks_per_seq, int32_t n_threads);

#ifdef __cplusplus
}
#endif
#endif /* PA_ORACLE_H */
