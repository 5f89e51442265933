// registry.hip - speaker identification against an enrolled registry on gfx950.
//
// Scores S = Q R^T for B query embeddings against N enrolled ones (D dims,
// f32), then keeps the k best rows per query.  Every product of two f32
// values is exact in f64 (24 + 24 significant bits) and the D products are
// summed in f64: the arithmetic of the reference's verify, whose distance is
// 1 - sum(ea * eb) accumulated in double (src/model.cpp:65-78), so a query's
// score for a row equals 1 - verify's distance for that pair up to the order
// of the f64 sum.  Ranking: highest score first, equal scores by the lower row
// index, so the result is deterministic.
//
// registry_tile_kernel: a workgroup scores a 64 x 256 (queries x rows)
// tile and writes each query's best k rows of it as candidates;
// registry_merge_kernel: one workgroup per query takes the best k of its
// ceil(N/256) * k candidates.
#include <cfloat>

#include "common.hpp"
#include "vdk.h"

namespace vdk {
namespace {

constexpr int kTQ = 64, kTR = 256, kDC = 32, kMaxK = 64, kMergeMax = 32;

// (s, i) ranks before (t, j): higher score, then lower index
__device__ __forceinline__ bool ranks_before(double s, int i, double t, int j) {
    return s > t || (s == t && i < j);
}

// Best (score, index) over `width` lanes (xor butterfly; width divides 64).
template <int WIDTH>
__device__ __forceinline__ void lane_best(double& s, int& i) {
#pragma unroll
    for (int off = WIDTH / 2; off > 0; off >>= 1) {
        const double os = __shfl_xor(s, off, WIDTH);
        const int oi = __shfl_xor(i, off, WIDTH);
        if (ranks_before(os, oi, s, i)) { s = os; i = oi; }
    }
}

// A workgroup scores 64 queries x 256 rows, 8 x 8 per thread (thread
// ty*32 + tx: queries 8*ty.., rows 8*tx..), over D in chunks of 32 staged
// through LDS as f32 (converted to f64 at use; the products are exact).
// Then the 32 threads of a query group (one half-wave) pick each of their 8
// queries' best k rows of the tile: k rounds of (each thread's best row that
// ranks after the previous pick, then a half-wave arg-max).
__global__ __launch_bounds__(256) void registry_tile_kernel(const float* __restrict__ q, int B,
                                                            const float* __restrict__ reg, int N, int D, int k,
                                                            double* __restrict__ cand_s, int* __restrict__ cand_i) {
    __shared__ __attribute__((aligned(16))) float sq[kDC][kTQ + 4];   // [dim][query]
    __shared__ __attribute__((aligned(16))) float sr[kDC][kTR + 4];   // [dim][row]
    const int tid = threadIdx.x, tx = tid & 31, ty = tid >> 5;
    const int q0 = blockIdx.y * kTQ, n0 = blockIdx.x * kTR;

    double acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = 0.0;

    for (int d0 = 0; d0 < D; d0 += kDC) {
        // 16-byte loads (D % 4 == 0), stored transposed
        for (int e = tid; e < kTQ * kDC / 4; e += 256) {
            const int r = e / (kDC / 4), c = (e - r * (kDC / 4)) * 4, d = d0 + c;
            const float4v v = (q0 + r < B && d < D) ? *reinterpret_cast<const float4v*>(q + (size_t)(q0 + r) * D + d)
                                                    : float4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < 4; ++t) sq[c + t][r] = v[t];
        }
        for (int e = tid; e < kTR * kDC / 4; e += 256) {
            const int r = e / (kDC / 4), c = (e - r * (kDC / 4)) * 4, d = d0 + c;
            const float4v v = (n0 + r < N && d < D) ? *reinterpret_cast<const float4v*>(reg + (size_t)(n0 + r) * D + d)
                                                    : float4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < 4; ++t) sr[c + t][r] = v[t];
        }
        __syncthreads();
#pragma unroll 2
        for (int c = 0; c < kDC; ++c) {
            const float4v a0 = *reinterpret_cast<const float4v*>(&sq[c][ty * 8]);
            const float4v a1 = *reinterpret_cast<const float4v*>(&sq[c][ty * 8 + 4]);
            const float4v b0 = *reinterpret_cast<const float4v*>(&sr[c][tx * 8]);
            const float4v b1 = *reinterpret_cast<const float4v*>(&sr[c][tx * 8 + 4]);
            double a[8], b[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                a[e] = a0[e]; a[e + 4] = a1[e];
                b[e] = b0[e]; b[e + 4] = b1[e];
            }
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[i][j] = fma(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }

    const int nchunks = gridDim.x;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int qq = q0 + ty * 8 + i;   // uniform over the half-wave
        if (qq >= B) break;
        double last_s = DBL_MAX;
        int last_i = -1;
        for (int r = 0; r < k; ++r) {
            double bs = -DBL_MAX;
            int bi = INT_MAX;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int row = n0 + tx * 8 + j;
                const double sj = acc[i][j];
                if (row < N && ranks_before(last_s, last_i, sj, row) && ranks_before(sj, row, bs, bi)) {
                    bs = sj;
                    bi = row;
                }
            }
            lane_best<32>(bs, bi);
            if (tx == 0) {
                const size_t o = ((size_t)qq * nchunks + blockIdx.x) * k + r;
                cand_s[o] = bs;
                cand_i[o] = bi;   // INT_MAX when the tile has fewer than k rows left
            }
            last_s = bs;
            last_i = bi;
        }
    }
}

// One workgroup per query: k rounds of a block-wide arg-max over the
// candidates that rank after the previous pick.  Up to 256 * kMergeMax
// candidates are held in registers (32 per thread); beyond that each round
// scans them in global memory.
__global__ __launch_bounds__(256) void registry_merge_kernel(const double* __restrict__ cand_s,
                                                             const int* __restrict__ cand_i, int ncand, int k,
                                                             int* __restrict__ out_i, float* __restrict__ out_s) {
    __shared__ double ws[4];
    __shared__ int wi[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, qq = blockIdx.x;
    const double* cs = cand_s + (size_t)qq * ncand;
    const int* ci = cand_i + (size_t)qq * ncand;
    const bool in_regs = ncand <= kMergeMax * 256;
    double mys[kMergeMax];
    int myi[kMergeMax];
#pragma unroll
    for (int m = 0; m < kMergeMax; ++m) {
        const int c = tid + m * 256;
        mys[m] = in_regs && c < ncand ? cs[c] : -DBL_MAX;
        myi[m] = in_regs && c < ncand ? ci[c] : INT_MAX;
    }
    double last_s = DBL_MAX;
    int last_i = -1;
    for (int r = 0; r < k; ++r) {
        double bs = -DBL_MAX;
        int bi = INT_MAX;
        if (in_regs) {
#pragma unroll
            for (int m = 0; m < kMergeMax; ++m)
                if (myi[m] != INT_MAX && ranks_before(last_s, last_i, mys[m], myi[m]) &&
                    ranks_before(mys[m], myi[m], bs, bi)) {
                    bs = mys[m];
                    bi = myi[m];
                }
        } else {
            for (int c = tid; c < ncand; c += 256) {
                const double sc = cs[c];
                const int ic = ci[c];
                if (ic != INT_MAX && ranks_before(last_s, last_i, sc, ic) && ranks_before(sc, ic, bs, bi)) {
                    bs = sc;
                    bi = ic;
                }
            }
        }
        lane_best<64>(bs, bi);
        if (lane == 0) { ws[wave] = bs; wi[wave] = bi; }
        __syncthreads();
        bs = ws[0];
        bi = wi[0];
#pragma unroll
        for (int w = 1; w < 4; ++w)
            if (ranks_before(ws[w], wi[w], bs, bi)) { bs = ws[w]; bi = wi[w]; }
        __syncthreads();
        if (tid == 0) {
            out_i[(size_t)qq * k + r] = bi;
            out_s[(size_t)qq * k + r] = (float)bs;
        }
        last_s = bs;
        last_i = bi;
    }
}

size_t workspace_bytes(int B, int N, int k) {
    const size_t nchunks = (size_t)(N + kTR - 1) / kTR;
    return (size_t)B * nchunks * k * (sizeof(double) + sizeof(int)) + 256;
}

}  // namespace
}  // namespace vdk

using namespace vdk;

extern "C" size_t vdk_registry_topk_workspace_size(int B, int N, int k) {
    if (B <= 0 || N <= 0 || k <= 0) return 0;
    return workspace_bytes(B, N, k);
}

extern "C" int vdk_registry_topk(const float* d_queries, int B, const float* d_registry, int N, int D, int k,
                                 void* d_work, size_t work_bytes, int* d_idx, float* d_score, void* stream) {
    return guarded([&] {
        require(d_queries && d_registry && d_work && d_idx && d_score, "registry_topk: NULL device pointer");
        require(B > 0 && N > 0 && D > 0, "registry_topk: empty queries or registry");
        require(D % 4 == 0 && (reinterpret_cast<uintptr_t>(d_queries) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(d_registry) & 15) == 0,
                "registry_topk: D must be a multiple of 4 and the embeddings 16-byte aligned");
        require(k >= 1 && k <= kMaxK, "registry_topk: k must be in 1..64");
        require(k <= N, "registry_topk: k exceeds the registry size");
        require((size_t)N * D < (1ull << 31) && (size_t)B * D < (1ull << 31), "registry_topk: registry too large");
        require(work_bytes >= workspace_bytes(B, N, k), "registry_topk: workspace too small");
        const int nchunks = (N + kTR - 1) / kTR;
        double* cand_s = static_cast<double*>(d_work);
        int* cand_i = reinterpret_cast<int*>(cand_s + (size_t)B * nchunks * k);
        hipStream_t s = static_cast<hipStream_t>(stream);
        hipLaunchKernelGGL(registry_tile_kernel, dim3(nchunks, cdiv(B, kTQ)), dim3(256), 0, s, d_queries, B,
                           d_registry, N, D, k, cand_s, cand_i);
        VDK_HIP(hipGetLastError());
        hipLaunchKernelGGL(registry_merge_kernel, dim3(B), dim3(256), 0, s, cand_s, cand_i, nchunks * k, k, d_idx,
                           d_score);
        VDK_HIP(hipGetLastError());
    });
}
