// Read-ceiling probe: a plain streaming read with no compute, timed by the
// benchmark on the same cold buffers as the GEMVs, so each GEMV's bandwidth
// can be set beside what a read of the same byte count reaches on this GPU.
// No counterpart in the reference (a measurement aid).
#include <hip/hip_runtime.h>
#include <stdint.h>


#include "../../include/tbhip_bench.h"
#include "gemv_common.hpp"
#include "tb_common.hpp"

namespace tb {
namespace {

using gemv::u32x4;

// Block b reads bytes [b * per, (b + 1) * per) of the total in passes of L
// non-temporal 16-byte loads per thread (all L in flight; the last pass is
// masked at the block's and the buffer's end), xor-folds them and writes one
// word per thread so the loads are not removed.
template <int L>
__global__ __launch_bounds__(256) void k_read_probe(const uint8_t *__restrict__ w, size_t per,
                                                    size_t total, uint32_t *__restrict__ out) {
    const size_t base = (size_t)blockIdx.x * per;
    u32x4 acc = {0u, 0u, 0u, 0u};
    const size_t pass = (size_t)L * 256 * 16;
    const size_t passes = (per + pass - 1) / pass;
    for (size_t r = 0; r < passes; ++r) {
        u32x4 v[L];
#pragma unroll
        for (int i = 0; i < L; ++i) {
            const size_t off = ((r * L + i) * 256 + threadIdx.x) * 16;
            v[i] = (off < per && base + off < total) ? gemv::load_nt16(w + base + off)
                                                     : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < L; ++i) acc ^= v[i];
    }
    out[(size_t)blockIdx.x * 256 + threadIdx.x] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

}  // namespace
}  // namespace tb

using namespace tb;

extern "C" int tb_read_probe(const void *buf, int64_t bytes, int64_t blocks, int64_t loads,
                             uint32_t *out, int64_t *bytes_read, void *stream) {
    {
        TB_REQUIRE(buf && out && bytes_read, TB_ERR_UNSUPPORTED,
                   "TB_UNSUPPORTED: read_probe: null pointer");
        TB_REQUIRE(((uintptr_t)buf & 15u) == 0 && blocks >= 1 && blocks <= (1 << 20) &&
                       (loads == 4 || loads == 8 || loads == 16),
                   TB_ERR_UNSUPPORTED,
                   "TB_UNSUPPORTED: read_probe: 16-byte aligned buffer, 1 <= blocks <= 2^20, "
                   "loads 4, 8 or 16");
        const size_t total = (size_t)bytes & ~(size_t)15;
        TB_REQUIRE(total >= 16, TB_ERR_UNSUPPORTED, "TB_UNSUPPORTED: read_probe: under 16 bytes");
        const size_t per = ((total + (size_t)blocks - 1) / (size_t)blocks + 15) & ~(size_t)15;
        *bytes_read = (int64_t)total;
        const auto st = static_cast<hipStream_t>(stream);
        const auto w = static_cast<const uint8_t *>(buf);
        const dim3 grid((unsigned)blocks), block(256);
        if (loads == 4)
            hipLaunchKernelGGL(k_read_probe<4>, grid, block, 0, st, w, per, total, out);
        else if (loads == 8)
            hipLaunchKernelGGL(k_read_probe<8>, grid, block, 0, st, w, per, total, out);
        else
            hipLaunchKernelGGL(k_read_probe<16>, grid, block, 0, st, w, per, total, out);
        TB_LAUNCHED();
        return TB_OK;
    }
}
