// The in-kernel stream-K finish protocol of mfma_tile.h (store_partial,
// finish_arrive, load_partial4) in a kernel of the same shape as the conv
// and GEMM epilogues: 64 partial floats per thread, the arrival, and the last
// workgroup summing every slot. Compiled to gfx950 assembly only (never
// run); tests/test_schedule.py reads the assembly and checks the order of
// the partial stores, their completion wait, the barriers, the counter
// atomic and the partial loads.
#include "mfma_tile.h"

__global__ void __launch_bounds__(256) finish_order_probe(float* ws, int* counter, float* out, int parts,
                                                          float scale) {
    const __amdgpu_buffer_rsrc_t rws = nnc::make_rsrc(ws);
    const uint32_t mine = (uint32_t)blockIdx.x * 64u * 256u * 4u;
#pragma unroll
    for (int r = 0; r < 64; ++r)
        nnc::store_partial(rws, mine + (uint32_t)(r * 256 + threadIdx.x) * 4u, scale * (float)(r + threadIdx.x));
    if (nnc::finish_arrive(counter, parts - 1)) {
        nnc::f32x4 v = {0.f, 0.f, 0.f, 0.f};
        for (int w = 0; w < parts; ++w)
            v += nnc::load_partial4(rws, (uint32_t)w * 64u * 256u * 4u + threadIdx.x * 16u);
        reinterpret_cast<nnc::f32x4*>(out)[threadIdx.x] = v;
    }
}
