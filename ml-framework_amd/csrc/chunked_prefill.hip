// chunked_prefill.hip -- chunked prefill (bf16 MFMA). Not yet implemented: returns
// PA_ERROR_UNSUPPORTED after validating its arguments.
#include "pa_internal.h"

extern "C" pa_status pa_chunked_prefill(pa_stream* stream, const pa_config* cfg, float* out,
                                        const void* q, const int32_t* q_start_loc,
                                        const int32_t* prefix_lens, const void* k_cache,
                                        const void* v_cache, const float* k_scale, const float* v_scale,
                                        const int32_t* block_tables, int32_t num_seqs,
                                        int32_t max_blocks_per_seq, int32_t max_chunk_len) {
    (void)stream; (void)out; (void)q; (void)q_start_loc; (void)prefix_lens; (void)k_cache;
    (void)v_cache; (void)k_scale; (void)v_scale; (void)block_tables; (void)num_seqs;
    (void)max_blocks_per_seq; (void)max_chunk_len;
    pa_status st = pa::check_config(cfg, "pa_chunked_prefill");
    if (st != PA_SUCCESS) return st;
    return pa::set_error(PA_ERROR_UNSUPPORTED, "pa_chunked_prefill: not implemented yet");
}
