/*
 * paged_attn.h -- C-ABI of libpa_hip.so, the MI355X (gfx950) paged-attention backend.
 *
 * The reference framework (werwedc/ml-framework, C#/.NET) reaches native code only through
 * P/Invoke declarations with CallingConvention.Cdecl into libraries it does not ship:
 *   - the CUDA runtime surface of its HAL   src/MLFramework/HAL/CUDA/CudaApi.cs:9-269
 *   - its custom-kernel library             src/MLFramework/HAL/CUDA/CudaKernels.cs:10-141
 *   - the paged-attention operator stub     src/MLFramework/Inference/PagedAttention/Kernels/
 *                                           CudaPagedAttentionKernel.cs:11-49 (throws)
 * Every entry point below replaces one of those declarations (cited per function) or fills the
 * operator stub. All functions are extern "C", take plain pointers and sizes, return a pa_status
 * (0 = success) and never throw. Launch functions validate their arguments on the host and return
 * an error without launching anything when a check fails. Device pointers are owned by the
 * caller; the library never frees memory it did not allocate through pa_alloc.
 *
 * Threading: launch functions are asynchronous on the given stream and return after enqueue. The
 * library keeps no mutable global state except a thread-local last-error string and the per-device
 * scratch array of pa_paged_decode_noalloc, so one pa_device may be driven from several host
 * threads, each with its own stream (pa_paged_decode_noalloc calls excepted: they share the scratch).
 */
#ifndef PAGED_ATTN_H
#define PAGED_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PA_API_VERSION_MAJOR 1
#define PA_API_VERSION_MINOR 1

/* Status codes. Mirrors the integer-error-to-exception mapping of the reference HAL
 * (src/MLFramework/HAL/CUDA/CudaError.cs, CudaException.CheckError used at CudaDevice.cs:15-21). */
typedef enum pa_status {
    PA_SUCCESS = 0,
    PA_ERROR_INVALID_ARGUMENT = 1,   /* null pointer, negative count, out-of-range value      */
    PA_ERROR_INVALID_CONFIG = 2,     /* pa_config inconsistent (heads, head_dim, block size)  */
    PA_ERROR_OUT_OF_MEMORY = 3,      /* device allocation failed                              */
    PA_ERROR_HIP = 4,                /* a HIP runtime call failed; see pa_get_last_error      */
    PA_ERROR_UNSUPPORTED = 5,        /* dtype / head_dim / GQA ratio not compiled             */
    PA_ERROR_WORKSPACE_TOO_SMALL = 6,/* caller workspace smaller than pa_*_workspace_size     */
    PA_ERROR_NO_DEVICE = 7           /* no HIP device with that ordinal                       */
} pa_status;

/* Element types. Values follow the order of MLFramework.Core.DataType only where they coincide
 * (src/MLFramework/Core/DataType.cs:6-21); the ABI fixes its own numbering. */
typedef enum pa_dtype {
    PA_DTYPE_FP32 = 0,
    PA_DTYPE_BF16 = 1,   /* stored as the upper 16 bits of fp32 (truncating conversion,
                            src/MLFramework/Amp/BFloat16.cs:99-117)                              */
    PA_DTYPE_INT8 = 2    /* symmetric int8 with an fp32 scale per (block, KV head)            */
} pa_dtype;

/* Attention phase, numbered as MlFramework.Inference.PagedAttention.Phases.AttentionPhase
 * (Phases/AttentionPhase.cs:6-17): Prefill = 0, Decode = 1. */
typedef enum pa_phase { PA_PHASE_PREFILL = 0, PA_PHASE_DECODE = 1 } pa_phase;

/* pa_config.flags */
#define PA_FLAG_NONE 0u
/* Chunked prefill: apply the reference's mask rule literally (mask only when phase == Decode and
 * the number of cached keys exceeds the number of queries, StandardPagedAttentionKernel.cs:57),
 * i.e. no mask when the prefix is empty or the phase is Prefill. Default: always causal. */
#define PA_FLAG_REFERENCE_LITERAL_MASK 1u
/* Chunked prefill: no mask at all -- the reference's Prefill phase, used by the dense
 * IPagedAttentionKernel interface when called with AttentionPhase.Prefill. */
#define PA_FLAG_NO_MASK 2u

/* Shape/dtype record passed by pointer to every launch function.
 * KV cache layout (per layer, K and V in separate buffers of kv_dtype), one tile per
 * (block, KV head) as in the reference's intended per-block tensor [layers, heads, blockSize,
 * headDim] (src/MLFramework/Inference/PagedAttention/Layers/PagedAttentionLayer.cs:315):
 *   K: [num_blocks][num_kv_heads][block_size][head_dim]   (token rows, row-major)
 *   V: [num_blocks][num_kv_heads][head_dim][block_size]   (dim rows: the tile is transposed so
 *      that P.V reads the 16 tokens of one dimension as one contiguous run)
 * int8 scales and running absolute maxima: fp32 [num_blocks][num_kv_heads], K and V separately. */
typedef struct pa_config {
    int32_t block_size;     /* tokens per physical block; 16 in every shipped configuration    */
    int32_t num_q_heads;    /* Hq                                                               */
    int32_t num_kv_heads;   /* Hkv; Hq % Hkv == 0, query head h reads KV head h / (Hq / Hkv)    */
    int32_t head_dim;       /* D: 64, 128 or 256; 32 for fp32 / bf16 caches (decode, append)  */
    int32_t kv_dtype;       /* pa_dtype of the cache                                            */
    int32_t q_dtype;        /* pa_dtype of Q and of the new K/V handed to pa_kv_append (FP32/BF16) */
    int32_t num_blocks;     /* physical blocks in the pool; ids outside [0, num_blocks) are
                               never dereferenced (decode/prefill read their tokens as zeros,
                               append skips their slots)                                        */
    float   scale;          /* softmax scale; <= 0 selects 1/sqrtf(head_dim)
                               (StandardPagedAttentionKernel.cs:18,28)                          */
    int32_t partition_size; /* decode split-K granularity in tokens; 0 = library default: the
                               batch's blocks are cut into one equal range per resident
                               workgroup (bf16/int8) or 256-token partitions (fp32). Otherwise a
                               multiple of 64 in [64, 4096] (bf16/int8) or 256/512 (fp32).      */
    uint32_t flags;         /* PA_FLAG_*                                                        */
    int32_t num_splits;     /* bf16/int8 decode: 0 = split by partition_size (above); P in
                               [1, 256] = every sequence's context is cut into P partitions of
                               whole blocks (ceil(blocks / P) each, fewer when the sequence has
                               fewer blocks), each streamed by its own worker per KV head and
                               merged with a log-sum-exp reduction -- the per-sequence split-K of
                               DecodeOrchestrator-style long-context decode. Requires
                               partition_size == 0; must be 0 for fp32 caches; the shared-prefix
                               decode ignores it.                                               */
} pa_config;

typedef struct pa_device pa_device;
typedef struct pa_stream pa_stream;
typedef struct pa_event pa_event;
typedef struct pa_graph pa_graph;

typedef struct pa_device_props {
    char name[256];
    char arch[64];             /* e.g. "gfx950:sramecc+:xnack-" */
    size_t total_memory;
    int32_t compute_units;
    int32_t ordinal;
} pa_device_props;

typedef enum pa_memcpy_kind {
    PA_MEMCPY_HOST_TO_HOST = 0,
    PA_MEMCPY_HOST_TO_DEVICE = 1,
    PA_MEMCPY_DEVICE_TO_HOST = 2,
    PA_MEMCPY_DEVICE_TO_DEVICE = 3,
    PA_MEMCPY_DEFAULT = 4
} pa_memcpy_kind;

/* ---- library / errors --------------------------------------------------------------------- */
pa_status pa_get_version(int32_t* major, int32_t* minor);
const char* pa_status_string(pa_status status);
/* Copies the calling thread's last error message (NUL-terminated, truncated to buf_len). */
pa_status pa_get_last_error(char* buf, size_t buf_len);

/* ---- device (replaces CudaApi.CudaGetDeviceCount/CudaSetDevice/CudaGetDeviceProperties/
 *      CudaDeviceSynchronize, CudaApi.cs:18-37;
 *      backs IDevice, src/MLFramework/HAL/IDevice.cs:6-42) ------------------------------------ */
pa_status pa_device_count(int32_t* count);
pa_status pa_device_open(int32_t ordinal, pa_device** out_device);
pa_status pa_device_close(pa_device* device);
pa_status pa_device_get_props(const pa_device* device, pa_device_props* props);
pa_status pa_device_synchronize(pa_device* device);

/* ---- memory (replaces CudaApi.CudaMalloc/CudaFree/CudaMemcpy/CudaMemset, CudaApi.cs:46-75;
 *      backs IMemoryAllocator/IMemoryBuffer, HAL/IMemoryAllocator.cs:6-43) ------------------- */
pa_status pa_alloc(pa_device* device, size_t bytes, void** dptr);
pa_status pa_free(pa_device* device, void* dptr);
/* Asynchronous on `stream` when it is non-null, otherwise synchronous. */
pa_status pa_memcpy(void* dst, const void* src, size_t bytes, int32_t kind, pa_stream* stream);
/* Refuses (PA_ERROR_INVALID_ARGUMENT) a stream that is capturing a graph: no memset is recorded. */
pa_status pa_memset(void* dst, int32_t value, size_t bytes, pa_stream* stream);

/* ---- streams and events (replace CudaApi.CudaStreamCreate/Destroy/Synchronize and
 *      CudaEventCreate/Destroy/Record/Query and CudaStreamWaitEvent, CudaApi.cs:81-128;
 *      back IStream/IEvent, HAL/IStream.cs:6-32, HAL/IEvent.cs:6-22) ---------------------- */
pa_status pa_stream_create(pa_device* device, pa_stream** out_stream);
/* Wraps an existing hipStream_t without taking ownership (interop with other HIP users). */
pa_status pa_stream_wrap(pa_device* device, void* hip_stream, pa_stream** out_stream);
pa_status pa_stream_native(const pa_stream* stream, void** hip_stream);
pa_status pa_stream_destroy(pa_stream* stream);
pa_status pa_stream_synchronize(pa_stream* stream);
pa_status pa_stream_wait_event(pa_stream* stream, pa_event* event);
pa_status pa_event_create(pa_device* device, pa_event** out_event);
pa_status pa_event_destroy(pa_event* event);
pa_status pa_event_record(pa_event* event, pa_stream* stream);
pa_status pa_event_query(pa_event* event, int32_t* completed);
pa_status pa_event_synchronize(pa_event* event);
pa_status pa_event_elapsed_ms(pa_event* start, pa_event* end, float* ms);

/* ---- graphs (replace the CUDA HAL's graph capture and replay: CUDAGraphCapture.BeginCapture /
 *      EndCapture, HAL/CUDA/Graphs/CUDAGraphCapture.cs:24-61, and CUDAGraph's instantiate /
 *      Execute / Validate / Dispose, HAL/CUDA/Graphs/CUDAGraph.cs:33-160) --------------------- */
/* Starts capturing the work enqueued on `stream` (thread-local capture mode, as the reference's
 * CaptureModeThreadLocal): launches made through this library on `stream` are recorded, not run,
 * until pa_graph_capture_end. `stream` must be a pa_stream (the null stream cannot capture). */
pa_status pa_graph_capture_begin(pa_stream* stream);
/* Ends the capture on `stream` and instantiates the graph; *out_graph replays the recorded work
 * with the same arguments (the same device buffers, whose contents the caller updates between
 * replays). On failure the capture is ended and no graph is returned. */
pa_status pa_graph_capture_end(pa_stream* stream, pa_graph** out_graph);
/* Replays the graph on `stream` (asynchronous). */
pa_status pa_graph_launch(pa_graph* graph, pa_stream* stream);
/* Number of nodes (kernel launches and copies) the graph holds. */
pa_status pa_graph_node_count(const pa_graph* graph, size_t* count);
pa_status pa_graph_destroy(pa_graph* graph);

/* ---- paged-attention operators (fill CudaPagedAttentionKernel.ComputePagedAttention,
 *      CudaPagedAttentionKernel.cs:24-36, behind IPagedAttentionKernel,
 *      Kernels/IPagedAttentionKernel.cs:11-34) ------------------------------------------------ */

/* Slot mapping for new tokens (device arrays). For sequence s, new token j (0 <= j < num_new[s])
 * sits at logical position p = start_pos[s] + j and gets
 *     slot_mapping[token_offset[s] + j] = block_tables[s][p / B] * B + p % B,
 * or -1 when that table entry is negative or p / B >= max_blocks_per_seq. This is the intended
 * BlockTable mapping (block k of a sequence holds tokens [k*B, (k+1)*B),
 * tests/MLFramework.Tests/Inference/PagedAttention/BlockTableTests.cs:115-134) combined with the
 * append position of PagedAttentionLayer.UpdateKVCache (Layers/PagedAttentionLayer.cs:256-272). */
pa_status pa_build_slot_mapping(pa_stream* stream, const pa_config* cfg,
                                const int32_t* block_tables, int32_t max_blocks_per_seq,
                                const int32_t* start_pos, const int32_t* num_new,
                                const int32_t* token_offset, int32_t num_seqs,
                                int32_t max_new_per_seq, int64_t* slot_mapping);

/* KV append / scatter (fills PagedAttentionLayer.UpdateKVCache/CopyTensorToBlock,
 * Layers/PagedAttentionLayer.cs:244-327, which is a no-op in the reference).
 * k_new, v_new: [n_tok][num_kv_heads][head_dim] of cfg->q_dtype (FP32 or BF16).
 * slot_mapping: [n_tok] int64, -1 = skip. Slots must be < num_blocks * block_size (others are
 *   skipped) and distinct: two new tokens of one call at one slot race.
 * FP32/BF16 caches store the converted value (fp32 -> bf16 truncates).
 * INT8 caches keep, per (block, KV head), an fp32 running absmax and scale = absmax / 127.
 *   Per call, the new tokens of one block raise absmax to max(absmax, max|x_new|); when it grows,
 *   every other slot of that block is requantised from q * old_scale with the new scale, then
 *   the new tokens are quantised with it. Quantisation is QuantizeSymmetric
 *   (src/MLFramework/Quantization/Operations/QuantizationOperations.cs:188-200).
 *   A block's new tokens may sit anywhere in the call's token list (split by other blocks'
 *   tokens or invalid slots); its segments (maximal runs of them) are applied in call order.
 *   The int8 append scans the slot list once per touched block (a workgroup per block finds
 *   whether an earlier token of the call owns its block), so its cost grows as blocks x n_tok:
 *   prompts above about 16k tokens are best appended in calls of at most that many tokens.
 *   k_scale/v_scale/k_absmax/v_absmax are required for INT8 and ignored otherwise. */
pa_status pa_kv_append(pa_stream* stream, const pa_config* cfg,
                       const void* k_new, const void* v_new,
                       const int64_t* slot_mapping, int32_t n_tok,
                       void* k_cache, void* v_cache,
                       float* k_scale, float* v_scale, float* k_absmax, float* v_absmax);

/* Bytes of device workspace pa_paged_decode / pa_paged_decode_append need for up to num_seqs
 * sequences of up to max_context_len tokens. bf16/int8 caches always need one (split partial
 * results and per-sequence offsets); fp32 caches only when a sequence spans several partitions
 * (else 0). The contents need no initialisation, and calls that share a workspace must not run
 * concurrently. */
pa_status pa_decode_workspace_size(const pa_config* cfg, int32_t num_seqs,
                                   int32_t max_context_len, size_t* bytes);

/* Ragged paged decode: one query token per sequence attends to its first context_lens[s] cached
 * tokens (the new token already appended), as DecodeOrchestrator.BatchDecode does with one
 * kernel call per sequence (Phases/DecodeOrchestrator.cs:64-109).
 *   out: [num_seqs][num_q_heads][head_dim] fp32
 *   q:   [num_seqs][num_q_heads][head_dim] of cfg->q_dtype
 *   block_tables: [num_seqs][max_blocks_per_seq] int32, context_lens: [num_seqs] int32
 *   max_context_len: host-side upper bound of context_lens (sizes the grid); tokens beyond it,
 *   or beyond max_blocks_per_seq * block_size, are not read. Tokens whose table entry lies
 *   outside [0, num_blocks) read as zero keys and values (never dereferenced).
 * Long sequences are split across workgroups (cfg->partition_size) and merged with a log-sum-exp
 * reduction through `workspace`. A sequence with context_len <= 0 produces zeros. */
pa_status pa_paged_decode(pa_stream* stream, const pa_config* cfg, float* out, const void* q,
                          const void* k_cache, const void* v_cache,
                          const float* k_scale, const float* v_scale,
                          const int32_t* block_tables, const int32_t* context_lens,
                          int32_t num_seqs, int32_t max_blocks_per_seq, int32_t max_context_len,
                          void* workspace, size_t workspace_bytes);

/* Fused decode layer-step: appends the token at position context_lens[s] - 1 of every sequence
 * (k_new/v_new [num_seqs][num_kv_heads][head_dim] of cfg->q_dtype) into the cache, then runs
 * pa_paged_decode. Cache bytes, int8 scales and absmax after the call are exactly those of
 * pa_kv_append with slot_mapping[s] = block_tables[s][(T-1)/16] * 16 + (T-1) % 16 followed by
 * pa_paged_decode; for bf16 caches both happen in one kernel (the rows stream their first T - 1
 * cached tokens and the new token joins each row's softmax from k_new / v_new, truncated to bf16 as
 * the cache stores it, while the wave that ends the row writes it into the cache), for int8 caches the
 * quantising append is a launch of its own ahead of the decode, and for fp32 caches a plain
 * copy kernel. No reference counterpart: the reference appends (PagedAttentionLayer.UpdateKVCache,
 * Layers/PagedAttentionLayer.cs:244-296) and decodes (DecodeOrchestrator.ComputeDecodeAttention,
 * Phases/DecodeOrchestrator.cs:64-80) in two steps; this is those two steps in one call.
 * Sequences with context_len <= 0 append nothing and produce zeros. */
pa_status pa_paged_decode_append(pa_stream* stream, const pa_config* cfg, float* out, const void* q,
                                 const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                                 float* k_scale, float* v_scale, float* k_absmax, float* v_absmax,
                                 const int32_t* block_tables, const int32_t* context_lens,
                                 int32_t num_seqs, int32_t max_blocks_per_seq, int32_t max_context_len,
                                 void* workspace, size_t workspace_bytes);

/* Bytes of device scratch the library holds per device for pa_paged_decode_noalloc. */
#define PA_NOALLOC_SCRATCH_BYTES (32u << 20)

/* pa_paged_decode for callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation): the same arguments without a workspace; the split-K
 * partials go to a device array of PA_NOALLOC_SCRATCH_BYTES that the library holds on each device
 * (resolved at pa_device_open, or at this call's first use on a device) until the process ends.
 * The call allocates nothing. It returns PA_ERROR_WORKSPACE_TOO_SMALL, launching nothing, when
 * pa_decode_workspace_size for the same shape exceeds PA_NOALLOC_SCRATCH_BYTES. Every call on a
 * device shares that device's array: calls that overlap on one device (two streams, two threads)
 * race. No counterpart in the reference: it serves the callers that cannot allocate. */
pa_status pa_paged_decode_noalloc(pa_stream* stream, const pa_config* cfg, float* out, const void* q,
                                  const void* k_cache, const void* v_cache,
                                  const float* k_scale, const float* v_scale,
                                  const int32_t* block_tables, const int32_t* context_lens,
                                  int32_t num_seqs, int32_t max_blocks_per_seq, int32_t max_context_len);

/* ---- Shared-prefix decode ----
 * Sequences forked from one parent share the parent's first physical blocks (copy-on-write:
 * the same block ids lead their tables; BlockShareManager.ShareBlock,
 * Inference/PagedAttention/Sharing/BlockShareManager.cs:34-54, keeps the refcounts). The result
 * is that of pa_paged_decode; the shared blocks are read once per group of up to 16 / G
 * sequences (G = num_q_heads / num_kv_heads) instead of once per sequence. No reference
 * counterpart: the reference decodes every sequence over its whole table. */

/* Bytes of the device plan for num_seqs sequences. */
pa_status pa_prefix_plan_bytes(int32_t num_seqs, size_t* bytes);

/* Builds the plan into `plan` (device memory, plan_bytes >= pa_prefix_plan_bytes) from the host
 * array shared_with_prev[num_seqs]: shared_with_prev[s] = number of leading block-table entries
 * sequence s has in common with sequence s - 1 (entry 0 is ignored; 0 = no link). Linked runs
 * are cut into groups of at most 16 / G sequences sharing the run's minimum link; *num_groups
 * receives the group count to pass to pa_paged_decode_prefix. The plan depends only on the
 * grouping, not on the context lengths, so it is rebuilt only when sequences fork or leave.
 * Synchronises `stream` (host-to-device copy); refused while the stream captures a graph. */
pa_status pa_prefix_plan_build(pa_stream* stream, const pa_config* cfg, int32_t num_seqs,
                               const int32_t* shared_with_prev, void* plan, size_t plan_bytes,
                               int32_t* num_groups);

/* The same plan written to host memory (plan_host, plan_bytes >= pa_prefix_plan_bytes), for a
 * caller that uploads it itself: int32 records {first sequence, members, shared blocks} for each
 * of the *num_groups groups, then {group or -1, shared blocks or 0} for each sequence. No GPU
 * call. */
pa_status pa_prefix_plan_fill(const pa_config* cfg, int32_t num_seqs, const int32_t* shared_with_prev,
                              int32_t* plan_host, size_t plan_bytes, int32_t* num_groups);

/* Workspace of pa_paged_decode_prefix for up to num_seqs sequences of up to max_context_len. */
pa_status pa_prefix_workspace_size(const pa_config* cfg, int32_t num_seqs, int32_t max_context_len,
                                   size_t* bytes);

/* pa_paged_decode over the same arguments plus a plan from pa_prefix_plan_build (same num_seqs
 * and head ratio). Contract: within a group the shared block ids are identical in every table
 * and every member's context_len covers the shared blocks (>= 16 * shared); a plan that breaks
 * it gives wrong attention but never reads outside the arguments. BF16 or INT8 caches;
 * num_seqs + num_groups <= 2047; cfg->partition_size is not used (equal ranges per worker). */
pa_status pa_paged_decode_prefix(pa_stream* stream, const pa_config* cfg, float* out, const void* q,
                                 const void* k_cache, const void* v_cache,
                                 const float* k_scale, const float* v_scale,
                                 const int32_t* block_tables, const int32_t* context_lens,
                                 int32_t num_seqs, int32_t max_blocks_per_seq, int32_t max_context_len,
                                 const void* plan, int32_t num_groups,
                                 void* workspace, size_t workspace_bytes);

/* Chunked prefill: prefill sequence s has chunk_len[s] = q_start_loc[s+1] - q_start_loc[s] new
 * query tokens at absolute positions prefix_lens[s] + i; the chunk's K/V must already be appended,
 * so keys are positions [0, prefix_lens[s] + chunk_len[s]) read through block_tables[s].
 * Query i attends to keys 0 .. prefix_lens[s] + i (bottom-right aligned causal mask,
 * StandardPagedAttentionKernel.cs:219-255); see PA_FLAG_REFERENCE_LITERAL_MASK.
 *   out: [total_q][num_q_heads][head_dim] fp32, q: [total_q][num_q_heads][head_dim] of
 *   cfg->q_dtype (BF16 or FP32); caches of any kv_dtype. BF16 and INT8 caches take head_dim 64,
 *   128 or 256 and compute on bf16 / fp16 MFMA operands; FP32 caches (head_dim 32 .. 256) compute
 *   in fp32 throughout (fp32 MFMA operands and accumulation), which is what the dense
 *   ComputePagedAttention of IPagedAttentionKernel (Kernels/IPagedAttentionKernel.cs:13-28) needs
 *   for more than one query: one launch over the prompt instead of one decode row per query.
 *   max_chunk_len: host-side upper bound of the chunk lengths.
 * Range: every finite cache value is accepted. The P.V product runs on fp16 operands; int8
 * caches fold log2 of each block's V scale into the softmax exponent, so P times the scale stays
 * within fp16 for any scale; bf16 caches whose V tiles hold a magnitude above 65504 (fp16's
 * largest) are detected as the tiles are converted, and the query tiles that read them are
 * computed again in fp32 (a slower path, taken only for such inputs). */
pa_status pa_chunked_prefill(pa_stream* stream, const pa_config* cfg, float* out, const void* q,
                             const int32_t* q_start_loc, const int32_t* prefix_lens,
                             const void* k_cache, const void* v_cache,
                             const float* k_scale, const float* v_scale,
                             const int32_t* block_tables, int32_t num_seqs,
                             int32_t max_blocks_per_seq, int32_t max_chunk_len);

/* ---- whole-block moves: copy-on-write and swap (the copy the reference leaves to a comment at
 *      beam divergence, BeamSearchBlockSharing.OnBeamDivergence, Sharing/BeamSearchBlockSharing.cs:
 *      69-79, over the refcounts of BlockShareManager.cs:34-105; and the block data moves of
 *      IPagedAttentionCache.GetBlockData / StoreBlockData, ContinuousBatching/KVCache/
 *      IPagedAttentionCache.cs:40-47, CacheBlockData.cs:7-12, which has no implementation) ----
 * Cache pointers (and the packed buffer) must be 16-byte aligned. int8 caches carry their
 * per-(block, KV head) k_scale, v_scale, k_absmax, v_absmax with the codes. */

/* Bytes of one packed block record: K of all KV heads (num_kv_heads * 16 * head_dim elements),
 * then V (same), then for int8 k_scale[Hkv], v_scale[Hkv], k_absmax[Hkv], v_absmax[Hkv] (fp32).
 * A multiple of 16. */
pa_status pa_block_bytes(const pa_config* cfg, size_t* bytes);
/* Copy-on-write: block_pairs [num_pairs][2] int32 (device) = (src, dst); every KV head's K and V
 * tiles (and int8 statistics) of block src are copied into block dst. Pairs with an id outside
 * [0, num_blocks) or src == dst are skipped. Within one call no block may be written twice, nor
 * be both a source and a destination. */
pa_status pa_copy_blocks(pa_stream* stream, const pa_config* cfg, void* k_cache, void* v_cache,
                         float* k_scale, float* v_scale, float* k_absmax, float* v_absmax,
                         const int32_t* block_pairs, int32_t num_pairs);
/* Swap-out: record i of `packed` ([n] records of pa_block_bytes, device memory; pa_memcpy moves
 * the records to and from host memory) receives block block_ids[i] (device int32), bit for bit.
 * Ids outside [0, num_blocks) are skipped (their records are not written). */
pa_status pa_gather_blocks(pa_stream* stream, const pa_config* cfg, const void* k_cache, const void* v_cache,
                           const float* k_scale, const float* v_scale, const float* k_absmax,
                           const float* v_absmax, const int32_t* block_ids, int32_t n, void* packed);
/* Swap-in: block block_ids[i] receives record i of `packed`, bit for bit (ids outside
 * [0, num_blocks) skipped; no block twice in one call). */
pa_status pa_scatter_blocks(pa_stream* stream, const pa_config* cfg, void* k_cache, void* v_cache,
                            float* k_scale, float* v_scale, float* k_absmax, float* v_absmax,
                            const int32_t* block_ids, int32_t n, const void* packed);
/* GetBlockData: tokens [0, tokens) (tokens <= 16) of block `block` as fp32, k_out / v_out
 * [tokens][num_kv_heads][head_dim] (device memory); bf16 widens exactly, int8 is code * scale.
 * k_scale/v_scale are needed for int8 only. */
pa_status pa_read_block_f32(pa_stream* stream, const pa_config* cfg, const void* k_cache, const void* v_cache,
                            const float* k_scale, const float* v_scale, int32_t block, int32_t tokens,
                            float* k_out, float* v_out);
/* StoreBlockData: tokens [0, tokens) of block `block` from fp32 k_in / v_in
 * [tokens][num_kv_heads][head_dim]; the cache bytes and int8 statistics afterwards are those of
 * pa_kv_append with fp32 input at slots block * 16 + t (row 0 is written, so an int8 block
 * starts afresh with scale = absmax of the new rows / 127). */
pa_status pa_write_block_f32(pa_stream* stream, const pa_config* cfg, void* k_cache, void* v_cache,
                             float* k_scale, float* v_scale, float* k_absmax, float* v_absmax,
                             int32_t block, int32_t tokens, const float* k_in, const float* v_in);

/* ---- the projections either side of attention (PagedAttentionLayer.ComputeAttention's
 *      _queryProj/_keyProj/_valueProj.Forward + UpdateKVCache and _outputProj.Forward,
 *      Layers/PagedAttentionLayer.cs:112-142; Linear.Forward y = x W^T without bias,
 *      Modules/Linear.cs:81-110). bf16 weights and activations (cfg->q_dtype must be BF16), fp32
 *      accumulation. Batches of at most 64 tokens (decode) run on a weight-streaming MFMA kernel
 *      with the k range split over workgroups (partials added in a fixed order, so results are
 *      deterministic); larger batches, operands not 16-byte aligned, a reduced dimension (hidden
 *      for Q/K/V, Hq * head_dim for O) not a multiple of 64, and output column counts not a
 *      multiple of 16 run on rocBLAS. The first rocBLAS call on a device creates
 *      its handle, so make one call of that shape before capturing these into a graph. ---- */

/* Bytes of workspace pa_qkv_project_append needs for n_tok tokens: for n_tok <= 64, the split
 * partials [splits][n_tok][(num_q_heads + 2 num_kv_heads) head_dim] fp32 (splits <= 8); above,
 * the fp32 GEMM output [n_tok][(num_q_heads + 2 num_kv_heads) head_dim]. Either way the GEMM
 * output y sits at the start of the workspace after the call. */
pa_status pa_qkv_workspace_size(const pa_config* cfg, int32_t n_tok, size_t* bytes);
/* x [n_tok][hidden] bf16; w_qkv [(Hq + 2 Hkv) * head_dim][hidden] bf16, the rows of Wq, then Wk,
 * then Wv. y = x w_qkv^T (fp32); q_out [n_tok][Hq][head_dim] (bf16) = y's Q columns truncated; the
 * K and V columns are appended into the cache at slot_mapping exactly as pa_kv_append does with
 * fp32 input (the int8 statistics included). */
pa_status pa_qkv_project_append(pa_stream* stream, const pa_config* cfg, const void* x, const void* w_qkv,
                                int32_t hidden, int32_t n_tok, const int64_t* slot_mapping, void* q_out,
                                void* k_cache, void* v_cache, float* k_scale, float* v_scale,
                                float* k_absmax, float* v_absmax, void* workspace, size_t workspace_bytes);
/* Bytes of workspace pa_o_project needs for n_tok tokens and `hidden` output columns: for
 * n_tok <= 64 the larger of the split partials [splits - 1][n_tok][hidden] fp32 and a bf16 copy
 * of the attention output; above, the bf16 copy. */
pa_status pa_o_workspace_size(const pa_config* cfg, int32_t hidden, int32_t n_tok, size_t* bytes);
/* attn [n_tok][Hq][head_dim] fp32 (the decode / prefill output), truncated to bf16;
 * w_o [hidden][Hq * head_dim] bf16; y [n_tok][hidden] fp32 = attn_bf16 w_o^T. */
pa_status pa_o_project(pa_stream* stream, const pa_config* cfg, const float* attn, const void* w_o,
                       int32_t hidden, int32_t n_tok, float* y, void* workspace, size_t workspace_bytes);

#ifdef __cplusplus
}
#endif

#endif /* PAGED_ATTN_H */
