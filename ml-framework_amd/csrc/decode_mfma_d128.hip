// decode_mfma_d128.hip -- the head_dim 128 instances of the MFMA paged-decode kernel.
#include "decode_mfma_launch.h"

template void pa::launch_decode_mfma<128>(pa::DecodeArgs&, int, bool, bool, bool, int, int64_t, hipStream_t);
