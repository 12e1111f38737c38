// decode_mfma_d32.hip -- the head_dim 32 instances of the MFMA paged-decode kernel (bf16 caches).
#include "decode_mfma_launch.h"

template void pa::launch_decode_mfma<32>(pa::DecodeArgs&, int, bool, bool, bool, int, int64_t, hipStream_t);
