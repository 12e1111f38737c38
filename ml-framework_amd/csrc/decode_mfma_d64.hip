// decode_mfma_d64.hip -- the head_dim 64 instances of the MFMA paged-decode kernel.
#include "decode_mfma_launch.h"

template void pa::launch_decode_mfma<64>(pa::DecodeArgs&, int, bool, bool, bool, int, int64_t, hipStream_t);
