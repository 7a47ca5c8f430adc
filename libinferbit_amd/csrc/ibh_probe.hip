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
//   ibh_probe_read: the same read with the launch shape as a parameter
//           (blocks, threads per block, 16-byte loads in flight per lane,
//           nontemporal or ordinary loads): block b reads its own contiguous
//           share, each wavefront 1 KB per load instruction, U instructions
//           issued before any result is used, then the next U.  Gives the
//           one-launch read ceiling the GEMV kernels are held against.
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

template <int U, bool NT>
__global__ __launch_bounds__(1024) void probe_read_shaped(const uint8_t* __restrict__ buf, size_t bytes, size_t share,
                                                          uint32_t* sink) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const size_t b0 = (size_t)blockIdx.x * share;
    const size_t b1 = b0 + share < bytes ? b0 + share : bytes;
    uint32_t a = 0;
    for (size_t off = b0 + (size_t)wave * U * 1024; off < b1; off += (size_t)nw * U * 1024) {
        uint4 v[U];
#pragma unroll
        for (int i = 0; i < U; i++) {
            const uint8_t* p = buf + min(off + (size_t)i * 1024 + 16 * lane, bytes - 16);
            if constexpr (NT) v[i] = ld_stream16(p);
            else v[i] = *(const uint4*)p;
        }
#pragma unroll
        for (int i = 0; i < U; i++) a ^= v[i].x + 3u * v[i].y + 5u * v[i].z + 7u * v[i].w;
    }
    if (a == 0x9e3779b9u && sink) sink[0] = a;
}

}  // namespace

extern "C" int ibh_probe_read(int blocks, int threads, int per_lane, int nontemporal, const void* buf, size_t bytes,
                              void* stream) {
    if (!buf || bytes < 16 || bytes % 16 || blocks < 1 || threads < 64 || threads > 1024 || threads % 64 ||
        (per_lane != 1 && per_lane != 2 && per_lane != 4 && per_lane != 8 && per_lane != 16)) {
        ibh_set_error("ibh_probe_read: bytes a multiple of 16 (>= 16), threads 64..1024 by 64, per_lane 1/2/4/8/16");
        return IBH_ERROR_PARAM;
    }
    hipStream_t st = ibh_resolve_stream(stream);
    const size_t share = ((bytes + blocks - 1) / blocks + 1023) / 1024 * 1024;
    const unsigned nb = (unsigned)((bytes + share - 1) / share);
#define IBH_PR(U_) do { if (nontemporal) probe_read_shaped<U_, true><<<nb, threads, 0, st>>>((const uint8_t*)buf, bytes, share, nullptr); \
                        else probe_read_shaped<U_, false><<<nb, threads, 0, st>>>((const uint8_t*)buf, bytes, share, nullptr); } while (0)
    switch (per_lane) {
    case 1: IBH_PR(1); break;
    case 2: IBH_PR(2); break;
    case 4: IBH_PR(4); break;
    case 8: IBH_PR(8); break;
    default: IBH_PR(16); break;
    }
#undef IBH_PR
    IBH_CHECK_LAUNCH("ibh_probe_read");
    return IBH_OK;
}

extern "C" int ibh_probe(int mode, const void* buf, size_t bytes, void* stream) {
    hipStream_t st = ibh_resolve_stream(stream);
    if (mode == 0) {
        probe_empty<<<256, 1024, 0, st>>>();
    } else if (mode == 1) {
        if (!buf || bytes < 16) {
            ibh_set_error("ibh_probe: buffer of < 16 bytes");
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
