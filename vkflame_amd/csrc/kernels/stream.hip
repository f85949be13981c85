// stream.hip — plain HBM read kernel, the measured read-bandwidth reference
// that the decode GEMVs' weight streams are compared with.
//
// Each wave reads 4 consecutive 1 KiB pieces per pass (lane = 16 bytes of
// each, 4 loads in flight per lane) and the waves of the grid stride over
// the buffer.  On MI355X, 256-thread workgroups, 4 per CU, gave the best
// rate of the launch shapes tried (1024-thread workgroups, 1 or 2 per CU,
// 8 or 16 loads in flight: 4-20 % slower).  Loads carry the non-temporal
// policy, as the GEMVs' weight loads do (39.8 MB: 7.60 -> 7.02 us; the
// fastest plain read found).  The loaded words are folded
// into one value that is stored only if it equals a constant, so the loads
// cannot be dropped and nothing is written in practice.
#include "vkf_device.h"

VKF_KERNEL void __launch_bounds__(256) vkf_stream_read(VkfStreamArgs a) {
    constexpr int U = 4;
    const vkf_u4 *p = (const vkf_u4 *)a.src;
    const uint64_t waves = (uint64_t)gridDim.x * 4;
    const uint64_t w = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63;
    uint32_t acc = 0;
    for (uint64_t base = w * U * 64; base < a.n16; base += waves * U * 64) {
        vkf_u4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint64_t i = base + u * 64 + lane;
            v[u] = i < a.n16 ? vkf_ld_nt<vkf_u4>(p + i) : vkf_u4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    if (acc == 0x9e3779b9u) a.sink[0] = acc;
}
