// ibh_probe.hip -- measurement probes with no counterpart in the reference:
// the per-launch floor of this part and the streaming rate of a plain read,
// the two numbers the matvec kernels' times are judged against.
//
//   mode 0: an empty kernel on the grid a 29 MB matvec launches (256 blocks
//           of 16 wavefronts): dispatch, wave launch and end-of-kernel cost.
//   mode 1: every byte of `buf` read once, 16 bytes per lane, 1 KB contiguous
//           per load instruction, 8 KB per wavefront, all loads issued before
//           any is used; nothing written (the sum is stored only if it equals
//           a value it cannot take for the synthetic data, so the loads stay).
#include "ibh_common.h"

using namespace ibh;

namespace {

__global__ __launch_bounds__(1024) void probe_empty() {}

__global__ __launch_bounds__(64) void probe_read(const uint8_t* __restrict__ buf, size_t bytes, uint32_t* sink) {
    constexpr int L = 8;
    const size_t base = ((size_t)blockIdx.x * L) * 1024 + 16 * (size_t)threadIdx.x;
    // unconditional loads of clamped addresses (a conditional load would sink
    // its use into a branch that waits for it before the next load issues)
    uint4 v[L];
#pragma unroll
    for (int i = 0; i < L; i++) v[i] = ld_stream16(buf + min(base + (size_t)i * 1024, bytes - 16));
    uint32_t a = 0;
#pragma unroll
    for (int i = 0; i < L; i++) a ^= v[i].x + 3u * v[i].y + 5u * v[i].z + 7u * v[i].w;
    if (a == 0x9e3779b9u && sink) sink[0] = a;
}

}  // namespace

extern "C" int ibh_probe(int mode, const void* buf, size_t bytes, void* stream) {
    hipStream_t st = ibh_resolve_stream(stream);
    if (mode == 0) {
        probe_empty<<<256, 1024, 0, st>>>();
    } else if (mode == 1) {
        if (!buf || !bytes) {
            ibh_set_error("ibh_probe: empty buffer");
            return IBH_ERROR_PARAM;
        }
        const size_t blocks = (bytes + 8 * 1024 - 1) / (8 * 1024);
        probe_read<<<(unsigned)blocks, 64, 0, st>>>((const uint8_t*)buf, bytes, nullptr);
    } else {
        ibh_set_error("ibh_probe: mode %d (0 empty, 1 read)", mode);
        return IBH_ERROR_PARAM;
    }
    IBH_CHECK_LAUNCH("ibh_probe");
    return IBH_OK;
}
