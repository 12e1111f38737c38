// decode_fp32.hip -- instantiations of the fp32-cache paged-decode kernel.
#include "decode_fp32.h"

namespace pa {
namespace {

template <int D, int G>
void launch_g(const DecodeArgs& a, dim3 grid, hipStream_t s) {
    if (a.part == 512) paged_decode_fp32_kernel<D, G, 512><<<grid, 256, 0, s>>>(a);
    else paged_decode_fp32_kernel<D, G, 256><<<grid, 256, 0, s>>>(a);
}

template <int D>
bool launch_d(const DecodeArgs& a, dim3 grid, hipStream_t s) {
    switch (a.group) {
        case 1: launch_g<D, 1>(a, grid, s); return true;
        case 2: launch_g<D, 2>(a, grid, s); return true;
        case 4: launch_g<D, 4>(a, grid, s); return true;
        case 8: launch_g<D, 8>(a, grid, s); return true;
        default: return false;
    }
}

}  // namespace

bool launch_decode_fp32(const DecodeArgs& a, int head_dim, dim3 grid, hipStream_t s) {
    switch (head_dim) {
        case 32: return launch_d<32>(a, grid, s);
        case 64: return launch_d<64>(a, grid, s);
        case 128: return launch_d<128>(a, grid, s);
        case 256: return launch_d<256>(a, grid, s);
        default: return false;
    }
}

}  // namespace pa
