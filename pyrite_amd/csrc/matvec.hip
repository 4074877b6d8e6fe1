// Fused GGML dequantize x matvec for gfx950: plain fp32 matvec entry points
// (VALU kernels of mv_kernel.h for batch chunks of 1-2, or any batch when the
// MFMA path does not apply; the MFMA matvec of mx.hip from batch 3, the MFMA
// dequant-GEMM of mg.hip from 16 where its estimate is lower).
#include <vector>

#include "mv_kernel.h"

namespace pyrite {

// From 16 vectors on, a quantized group goes through whichever of the MFMA
// dequant-GEMM and the chunked MFMA matvec this estimate makes faster (us;
// constants fitted to MI355X timings of 2048x1024 Q3_K, 14336x4096 Q4_K and
// 4096x14336 Q6_K at 16-128 vectors):
//   GEMM:   10 (+ 6 for the reduce launch of a split-K launch) + (3.2 for
//           Q4_K, 4.8 otherwise) x the blocks one workgroup walks (a row's
//           blocks, or its K part's when the launch splits K to fill the
//           CUs), per pass of up to 256 workgroups;
//   matvec: 5 + per 8-token chunk max(3, weight bytes / 2 TB/s) (weights
//           read once, each chunk's MFMAs over the parked weights).
constexpr size_t kGemmMinBatch = 16;

static bool gemm_faster(int type, const TypeGeo& g, const MatvecArgs* mats, size_t n, size_t batch) {
    if (batch < kGemmMinBatch) return false;
    size_t max_cols = 0;
    for (size_t i = 0; i < n; ++i)
        if (mats[i].cols > max_cols) max_cols = mats[i].cols;
    double bytes = 0.0;
    for (size_t i = 0; i < n; ++i) bytes += (double)mats[i].rows * (double)(mats[i].cols / g.bs * g.bpb);
    // per-block cost in units of one 256-column super-block
    const double per_blk = (type == T_Q4_K ? 3.2 : 4.8) * (double)g.bs / 256.0;
    int kblocks = 0;
    const long long wgs = mg_workgroups(type, mats, n, batch, &kblocks);
    const bool split = kblocks * g.bs < (int)(max_cols);
    const double t_gemm = 10.0 + (split ? 6.0 : 0.0) + per_blk * (double)kblocks * (double)((wgs + 255) / 256);
    const double chunk = bytes / 2e6 > 3.0 ? bytes / 2e6 : 3.0;
    const double t_mx = 5.0 + chunk * (double)((batch + 7) / 8);
    return t_gemm < t_mx;
}

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
    if (mfma && batch >= 3) {
        // Each matrix takes the path its own estimate picks, so a grouped
        // launch computes every matrix exactly as a launch of it alone: the
        // dequant-GEMM part (matrices sharing activations share a launch),
        // then the MFMA matvec part (every 8-token chunk in one launch).
        std::vector<MatvecArgs> gm, vm;
        for (size_t i = 0; i < n; ++i) (gemm_faster(type, g, mats + i, 1, batch) ? gm : vm).push_back(mats[i]);
        if (!gm.empty()) {
            const int rc = mg_group_launch(type, gm.data(), gm.size(), batch, al, stream, start, vm.empty() ? stop : nullptr);
            if (rc) return rc;
        }
        if (!vm.empty())
            return mx_group_launch(type, vm.data(), vm.size(), batch, 0, al, stream, gm.empty() ? start : nullptr, stop);
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
