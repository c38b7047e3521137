// fp32 GEMM on CDNA4 matrix cores for the three contractions of a linear
// layer's training step:
//   forward  Y  = X . W        (trans_a = 0, trans_b = 0)
//   backward dX = dY . W^T     (trans_a = 0, trans_b = 1)
//   backward dW = X^T . dY     (trans_a = 1, trans_b = 0)
// The reference materialises W^T and X^T with t().contiguous() before its
// blocked CPU kernel (grad_fn/ops/matmul.rs:68-80, transform/contiguous.rs);
// here the transpose is only a different index order in the global->LDS
// staging, so no transposed copy ever exists.
//
// Tiling: a 256-thread workgroup (4 wave64, 2x2) owns a 128x128 tile of C and
// walks K in steps of 16.  Each wave owns 64x64 = 2x2 blocks of
// v_mfma_f32_32x32x2_f32 accumulators (64 fp32 per lane).  Operand tiles live
// in LDS k-major (As[k][m], Bs[k][n]) so that the MFMA operand read of a
// wave is two rows of 32 consecutive floats; odd k rows are stored with the
// two 32-column halves swapped so those two rows fall in different banks.
// LDS is double buffered: global loads for tile k+1 are issued before the
// MFMAs of tile k and written to the other buffer after them, with one
// barrier per K step.
// Workgroups are renumbered so that each XCD (the hardware deals workgroups
// round-robin over 8 XCDs, each with its own L2) receives a contiguous run of
// tiles, ordered in groups of 8 tile-rows so neighbouring tiles share A rows
// and B columns in that L2.
#include "ts_hip_internal.h"

namespace tship {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 16;
constexpr int kGroupM = 8;
constexpr int kXcds = 8;

__device__ inline int swz(int k) { return (k & 1) << 5; }

struct GemmArgs {
    const float *A;
    const float *B;
    float *C;
    long M, N, K, lda, ldb, ldc;
    int tiles_m, tiles_n;
    bool a_vec, b_vec;  // 16-byte aligned base and leading dimension
};

// Stage one operand tile (logical [BK][128] slice, k-major) into registers.
// KCONTIG: the operand's k index is contiguous in memory (row-major A, or
// B^T); otherwise the 128-wide index (m of A, n of B) is contiguous.
template <bool KCONTIG>
__device__ inline void load_tile(const float *__restrict__ P, long ld, long rows, long K,
                                 long r0, long k0, bool vec_ok, float4 (&reg)[2]) {
    const int t = threadIdx.x;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        if (KCONTIG) {
            const int row = (t >> 2) + 64 * s, kq = t & 3;
            const long gr = r0 + row, gk = k0 + 4 * kq;
            if (vec_ok && gr < rows && gk + 3 < K) {
                reg[s] = *reinterpret_cast<const float4 *>(P + gr * ld + gk);
            } else {
                float v[4];
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    v[c] = (gr < rows && gk + c < K) ? P[gr * ld + gk + c] : 0.0f;
                reg[s] = make_float4(v[0], v[1], v[2], v[3]);
            }
        } else {
            const int kk = (t >> 5) + 8 * s, q = t & 31;
            const long gk = k0 + kk, gr = r0 + 4 * q;
            if (vec_ok && gk < K && gr + 3 < rows) {
                reg[s] = *reinterpret_cast<const float4 *>(P + gk * ld + gr);
            } else {
                float v[4];
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    v[c] = (gk < K && gr + c < rows) ? P[gk * ld + gr + c] : 0.0f;
                reg[s] = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    }
}

template <bool KCONTIG>
__device__ inline void store_tile(float (*S)[128], const float4 (&reg)[2]) {
    const int t = threadIdx.x;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        if (KCONTIG) {
            const int row = (t >> 2) + 64 * s, kq = t & 3;
            const float *v = reinterpret_cast<const float *>(&reg[s]);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int k = 4 * kq + c;
                S[k][row ^ swz(k)] = v[c];
            }
        } else {
            const int kk = (t >> 5) + 8 * s, q = t & 31;
            *reinterpret_cast<float4 *>(&S[kk][(4 * q) ^ swz(kk)]) = reg[s];
        }
    }
}

// Tile coordinates of this workgroup (see the file comment).
__device__ inline void tile_coords(int tiles_m, int tiles_n, int &tm, int &tn) {
    const int G = tiles_m * tiles_n;
    const int b = blockIdx.x;
    const int xcd = b % kXcds;
    int prefix = 0;
    for (int y = 0; y < xcd; ++y) prefix += (G - y + kXcds - 1) / kXcds;
    const int logical = prefix + b / kXcds;
    const int group_size = kGroupM * tiles_n;
    const int group = logical / group_size;
    const int first_m = group * kGroupM;
    int gsz = tiles_m - first_m;
    if (gsz > kGroupM) gsz = kGroupM;
    const int in_group = logical - group * group_size;
    tm = first_m + in_group % gsz;
    tn = in_group / gsz;
}

template <bool TA, bool TB>
__global__ __launch_bounds__(256) void gemm_f32_mfma(GemmArgs g) {
    __shared__ float As[2][BK][BM];
    __shared__ float Bs[2][BK][BN];

    int tm, tn;
    tile_coords(g.tiles_m, g.tiles_n, tm, tn);
    const long i0 = static_cast<long>(tm) * BM, j0 = static_cast<long>(tn) * BN;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lrow = lane & 31, lhalf = lane >> 5;

    floatx16 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;

    const long nk = (g.K + BK - 1) / BK;
    float4 ra[2], rb[2];
    // A is "k-contiguous" unless transposed; B is k-contiguous only when transposed.
    load_tile<!TA>(g.A, g.lda, g.M, g.K, i0, 0, g.a_vec, ra);
    load_tile<TB>(g.B, g.ldb, g.N, g.K, j0, 0, g.b_vec, rb);
    store_tile<!TA>(As[0], ra);
    store_tile<TB>(Bs[0], rb);
    __syncthreads();

    for (long kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) {
            load_tile<!TA>(g.A, g.lda, g.M, g.K, i0, (kt + 1) * BK, g.a_vec, ra);
            load_tile<TB>(g.B, g.ldb, g.N, g.K, j0, (kt + 1) * BK, g.b_vec, rb);
        }
#pragma unroll
        for (int s = 0; s < BK / 2; ++s) {
            const int k = 2 * s + lhalf;
            float af[2], bf[2];
#pragma unroll
            for (int a = 0; a < 2; ++a) af[a] = As[cur][k][(wm * 64 + a * 32 + lrow) ^ swz(k)];
#pragma unroll
            for (int b = 0; b < 2; ++b) bf[b] = Bs[cur][k][(wn * 64 + b * 32 + lrow) ^ swz(k)];
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[a], bf[b], acc[a][b], 0, 0, 0);
        }
        if (more) {
            store_tile<!TA>(As[cur ^ 1], ra);
            store_tile<TB>(Bs[cur ^ 1], rb);
        }
        __syncthreads();
    }

    // Accumulator layout of v_mfma_f32_32x32x2_f32: lane l, register r holds
    // C[8*(r/4) + 4*(l/32) + r%4][l%32] of the 32x32 block.
#pragma unroll
    for (int a = 0; a < 2; ++a) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const long j = j0 + wn * 64 + b * 32 + lrow;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const long i = i0 + wm * 64 + a * 32 + 8 * (r >> 2) + 4 * lhalf + (r & 3);
                if (i < g.M && j < g.N) g.C[i * g.ldc + j] = acc[a][b][r];
            }
        }
    }
}

}  // namespace tship

using namespace tship;

extern "C" int ts_hip_gemm(int trans_a, int trans_b, size_t M, size_t N, size_t K, const float *A,
                           size_t lda, const float *B, size_t ldb, float *C, size_t ldc,
                           void *stream) {
    if (M == 0 || N == 0) return TS_HIP_OK;
    if (!C || ldc < N) return TS_HIP_EINVAL;
    if (K == 0) {  // empty contraction: C = 0
        if (ldc != N) return TS_HIP_EINVAL;
        return ts_hip_fill(C, 0.0f, M * N, stream);
    }
    if (!A || !B) return TS_HIP_EINVAL;
    if (lda < (trans_a ? M : K) || ldb < (trans_b ? K : N)) return TS_HIP_EINVAL;
    const size_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    if (tiles_m * tiles_n > 0x7fffffffULL || M > 0x3fffffffffffULL) return TS_HIP_EINVAL;
    GemmArgs g;
    g.A = A; g.B = B; g.C = C;
    g.M = static_cast<long>(M); g.N = static_cast<long>(N); g.K = static_cast<long>(K);
    g.lda = static_cast<long>(lda); g.ldb = static_cast<long>(ldb); g.ldc = static_cast<long>(ldc);
    g.tiles_m = static_cast<int>(tiles_m);
    g.tiles_n = static_cast<int>(tiles_n);
    g.a_vec = aligned16(A) && (lda % 4 == 0);
    g.b_vec = aligned16(B) && (ldb % 4 == 0);
    dim3 grid(static_cast<unsigned>(tiles_m * tiles_n)), block(256);
    hipStream_t s = as_stream(stream);
    if (!trans_a && !trans_b) hipLaunchKernelGGL((gemm_f32_mfma<false, false>), grid, block, 0, s, g);
    else if (!trans_a && trans_b) hipLaunchKernelGGL((gemm_f32_mfma<false, true>), grid, block, 0, s, g);
    else if (trans_a && !trans_b) hipLaunchKernelGGL((gemm_f32_mfma<true, false>), grid, block, 0, s, g);
    else hipLaunchKernelGGL((gemm_f32_mfma<true, true>), grid, block, 0, s, g);
    return launch_status();
}

extern "C" int ts_hip_matmul(const float *a, const float *b, float *c, size_t m, size_t n, size_t k,
                             void *stream) {
    return ts_hip_gemm(0, 0, m, n, k, a, k, b, n, c, n, stream);
}
