// Fused GGML dequantize x matvec for gfx950: plain fp32 matvec entry points
// (VALU kernels of mv_kernel.h for batch chunks of 1-2, or any batch when the
// MFMA path does not apply; MFMA kernels of mx.hip for batch >= 3).
#include "mv_kernel.h"

namespace pyrite {

// From this many vectors on, quantized matrices go through the GEMM kernel.
constexpr size_t kGemmMinBatch = 64;

int matvec_group_launch(int type, const MatvecArgs* mats, size_t n, size_t batch, hipStream_t stream,
                        hipEvent_t start, hipEvent_t stop) {
    const TypeGeo g = type_geo(type);
    bool al = false;
    size_t max_cols = 0;
    if (const int rc = validate_group(g, mats, n, batch, &al, &max_cols)) return rc;
    const bool forced = matvec_path_env() == 'v';
    // the MFMA kernels address a 32-row tile's weights with 32-bit offsets
    const bool mfma = g.bs > 1 && !forced && mx_type_supported(type) &&
                      32ull * (max_cols / g.bs * g.bpb) + 16 < 0x7FFFFFFFull;
    // prefill-sized batches: the MFMA dequant-GEMM (matrices sharing activations share a launch)
    if (mfma && batch >= kGemmMinBatch) return mg_group_launch(type, mats, n, batch, al, stream, start, stop);
    if (mfma && batch >= 3) {
        for (size_t done = 0; done < batch; done += 8) {
            const size_t c = batch - done < 8 ? batch - done : 8;
            const int rc = mx_group_launch(type, mats, n, c, done, al, stream, done == 0 ? start : nullptr,
                                           done + c >= batch ? stop : nullptr);
            if (rc != 0) return rc;
        }
        return 0;
    }
    return valu_group_launch<false>(type, g, al, mats, nullptr, n, batch, max_cols, stream, start, stop);
}

int matvec_launch(int type, const uint8_t* W, size_t w_len, size_t rows, size_t cols, const float* X, size_t ldx,
                  float* Y, size_t ldy, size_t batch, hipStream_t stream) {
    MatvecArgs m{W, w_len, rows, cols, X, ldx, Y, ldy};
    return matvec_group_launch(type, &m, 1, batch, stream, nullptr, nullptr);
}

}  // namespace pyrite
