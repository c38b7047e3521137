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
// Tiling.  A workgroup owns a BM x BN tile of C and walks K in steps of BK=16.
// Its waves form a WM x WN grid; each wave owns (BM/WM) x (BN/WN) of C as a
// grid of 32x32 v_mfma_f32_32x32x2_f32 accumulators.  Two shapes:
//   large problems: 256x256 tiles, 8 waves (2 per SIMD), 128x64 per wave;
//   smaller problems: 128x128 tiles, 4 waves, 64x64 per wave;
//   small problems (fewer 128x128 tiles than half the CUs): 64x64 tiles,
//   4 waves of one 32x32 accumulator each; when even those are fewer than a
//   quarter of the CUs and K >= 512 (the README and config-4 shapes with
//   M = 32 or N = 10), K is split into up to 16 slices computed as a batch
//   into a stream-ordered temporary and added in slice order afterwards.
// LDS holds each operand tile k-major (As[k][m], Bs[k][n]) so a wave's MFMA
// operand read is two rows of 32 consecutive floats.  Columns are XOR-swizzled
// per k row (swz) so that (a) the two rows an MFMA operand read touches fall
// in different bank halves and (b) the transposing store of a k-contiguous
// operand (16 rows x 4 k-quads per wave instruction) is bank-conflict free.
// Pipeline: LDS double buffer; at the top of iteration kt the registers of
// tile kt+1 go to LDS and the global loads of tile kt+2 are issued, so both
// overlap the MFMAs of tile kt; one barrier per K step.  Tiles wholly inside
// the matrices (a uniform test) take an unguarded dwordx4 path; edge tiles
// load element by element with bounds checks.
// Workgroups are renumbered so that each XCD (the hardware deals workgroups
// round-robin over 8 XCDs, each with its own L2) receives a contiguous run of
// tiles, ordered in groups of 8 tile-rows so neighbouring tiles share A rows
// and B columns in that L2.
//
// Operand transforms (ts_hip_gemm_*_xf): the register-staged tiles, the
// narrow and one-k-tile kernels and the column strips can apply a short
// elementwise chain to an operand as they load it (in registers, before the
// LDS store or the MFMA), in instantiations of their own (XF), so a deferred
// gradient such as relu's backward of a constant is never stored.
//
// Large aligned problems (both operands 16-byte aligned, leading dimensions
// % 4 == 0, enough 256x256 tiles to fill the chip) take gemm_f32_lds_dma
// instead: operand tiles go from global memory straight into LDS with
// global_load_lds_dwordx4 (no VGPR staging, no ds_write), and the MFMA
// operands of the next two k-steps are read from LDS while the MFMAs of the
// current two run, across tile boundaries too.  Its k order per MFMA differs
// (k of step s, lane half h = 4*(s/2) + 2h + s%2) so that a k-contiguous
// operand gives two steps' values in one 8-byte LDS read.
#include <cstring>
#include <mutex>
#include <vector>

#include "ts_hip_internal.h"

namespace tship {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 16;
constexpr int kGroupM = 8;
constexpr int kXcds = 8;

// Column swizzle of LDS row k: bit 4 from the k-quad, bit 5 from k's parity.
__device__ __forceinline__ int swz(int k) { return (((k >> 2) & 3) << 4) ^ ((k & 1) << 5); }

constexpr int kMaxBatchRank = 6;

// An elementwise transform of one operand, applied to each element as it is
// loaded (ts_hip_operand_xf; n == 0: none).  It maps +0 to +0, so the zeros
// that pad a partial k tile stay zeros.
struct OperandXf {
    int n;
    uint8_t code[TS_HIP_XF_MAX_OPS];
    float imm[TS_HIP_XF_MAX_OPS];
};

// A transform read once into scalar registers (the op codes packed in one
// word), so applying it reads no memory.
struct XfRegs {
    int n;
    uint32_t codes;
    float c0, c1, c2, c3;
};
__device__ __forceinline__ XfRegs xf_load(const OperandXf &x) {
    XfRegs r;
    r.n = x.n;
    r.codes = static_cast<uint32_t>(x.code[0]) | (static_cast<uint32_t>(x.code[1]) << 8) |
              (static_cast<uint32_t>(x.code[2]) << 16) | (static_cast<uint32_t>(x.code[3]) << 24);
    r.c0 = x.imm[0];
    r.c1 = x.imm[1];
    r.c2 = x.imm[2];
    r.c3 = x.imm[3];
    return r;
}

// The ops of the transform in order on every element (at(e), E of them),
// each one fp32 operation as the elementwise kernel of the same op computes
// it.  The op's case is chosen once per op (a uniform branch) with the
// elements looped inside it: a switch per element multiplied the kernels'
// code (and compile time) by the element count.
#define TS_XF_EACH(expr) \
    _Pragma("unroll") for (int e = 0; e < E; ++e) { float &x = at(e); x = (expr); } break
template <int E, class At>
__device__ __forceinline__ void xf_each(const XfRegs &xf, At &&at) {
    for (int i = 0; i < xf.n; ++i) {  // uniform
        const uint32_t code = (xf.codes >> (8 * i)) & 255u;
        const float c = i == 0 ? xf.c0 : i == 1 ? xf.c1 : i == 2 ? xf.c2 : xf.c3;
        switch (code) {
            case TS_HIP_XF_ADD_S: TS_XF_EACH(x + c);
            case TS_HIP_XF_SUB_S: TS_XF_EACH(x - c);
            case TS_HIP_XF_MUL_S: TS_XF_EACH(x * c);
            case TS_HIP_XF_DIV_S: TS_XF_EACH(x / c);
            case TS_HIP_XF_RSUB_S: TS_XF_EACH(c - x);
            case TS_HIP_XF_RDIV_S: TS_XF_EACH(c / x);
            case TS_HIP_XF_RELU: TS_XF_EACH(x > 0.0f ? x : 0.0f);
            case TS_HIP_XF_RELU_BWD_S: TS_XF_EACH(x > 0.0f ? c : 0.0f);
            default: TS_XF_EACH(x * x);  // TS_HIP_XF_SQUARE
        }
    }
}
#undef TS_XF_EACH

template <int N>
__device__ __forceinline__ void xf_array(const XfRegs &xf, float (&v)[N]) {
    if (xf.n) xf_each<N>(xf, [&](int e) -> float & { return v[e]; });
}

template <int NF>
__device__ __forceinline__ void xf_regs(const XfRegs &xf, f4v_t (&reg)[NF]) {
    if (!xf.n) return;  // uniform
    float v[4 * NF];
#pragma unroll
    for (int e = 0; e < 4 * NF; ++e) v[e] = reg[e / 4][e % 4];
    xf_each<4 * NF>(xf, [&](int e) -> float & { return v[e]; });
#pragma unroll
    for (int e = 0; e < 4 * NF; ++e) reg[e / 4][e % 4] = v[e];
}

struct GemmArgs {
    const float *A;
    const float *B;
    float *C;
    int M, N, K, lda, ldb, ldc;
    int tiles_m, tiles_n;
    int vec;  // both operands 16-byte aligned with leading dimensions % 4 == 0
    // Batched form (batch_rank > 0): workgroup b computes tile b % tiles of
    // batch b / tiles; a batch's coordinates (row-major over bdims) select
    // A + sum(c_k * sa[k]) and B + sum(c_k * sb[k]) (0 strides on broadcast
    // axes), and C + batch * sc.
    int batch_rank;
    int tiles;  // tiles_m * tiles_n
    int bdims[kMaxBatchRank];
    long long sa[kMaxBatchRank], sb[kMaxBatchRank];
    long long sc;
    // Epilogue (plain form only; all null / 0 for a bare product): the stored
    // value is the product, plus bias[j] when bias is set, then v > 0 ? v : +0 as
    // relu does when relu is set, then kept only where mask[i*ldc + j] > 0
    // (relu's backward with its saved output) when mask is set.
    const float *bias;
    const float *mask;
    int relu;
    // Column sums of B (trans_b == 0; the bias gradient beside a weight
    // gradient) in the column sum's fixed order.  The LDS-DMA kernel writes
    // the sum of each chunk of kColsumRows rows to colsum_part[chunk][n] (f64)
    // from the B tiles it stages anyway -- chunk c by the workgroups of tile
    // row c % tiles_m, so the work is spread over the grid -- and a pass after
    // the product adds the chunks into colsum[n]; the register-staged tiles
    // append a workgroup per 16 columns to their grid, the narrow kernel's
    // first workgroup and the skinny kernel's slice sum add B's columns as
    // they go.  Null: none.
    float *colsum;
    double *colsum_part;
    int kslice;  // skinny: k rows per slice
    // operand transforms (register-staged tiles, the narrow and one-k-tile
    // kernels and the column strips apply them; the others take none)
    OperandXf xa, xb;
    // The sum (mean: / (float)sum_n) of the sum_n floats at sum_x, each put
    // through sum_xf first, into sum_out[0] with the bits of ts_hip_sum over
    // the transformed values: one workgroup appended to the grid of a product
    // with column sums (after the register-staged tiles' strips, or as the
    // narrow kernel's last row block) runs sum_in_workgroup over sum_blocks
    // first-pass workgroups.  Null sum_out: none.
    const float *sum_x;
    float *sum_out;
    size_t sum_n;
    int sum_mean, sum_blocks;
    OperandXf sum_xf;
    // Epilogue subtraction (narrow kernel only): after the bias, v = v -
    // sub[i*ldc + j] (laid out as C).  Null: none.
    const float *sub;
};

// Store of a wave's FM x FN accumulator blocks, the wave tile's corner at
// (i0, j0).  Accumulator layout of v_mfma_f32_32x32x2_f32: lane l, register
// r holds C[8*(r/4) + 4*(l/32) + r%4][l%32] of the 32x32 block.  With EPI the
// stored value is the product, plus bias[j], then v > 0 ? v : +0 (relu), then
// kept only where mask[i*ldc + j] > 0: the unfused ops in their order.  A row
// of blocks at a time: its mask is loaded before its first store, so those
// loads overlap each other (every block's at once would need a register per
// output element).  EPI is one of the kinds below; kEpiBiasRelu ignores
// the mask, so a kernel that never sees one keeps no registers for it.
enum : int { kEpiNone = 0, kEpiBiasRelu = 1, kEpiAll = 2 };
// s_waitcnt immediate for vmcnt(0) with expcnt and lgkmcnt left at their
// maxima (gfx9 encoding: vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8]).
constexpr int kWaitVm0 = 0x0F70;

template <int EPI, int FM, int FN>
__device__ __forceinline__ void store_tile(const GemmArgs &g, const floatx16 (&acc)[FM][FN], float *Cp, int i0,
                                           int j0, int lrow, int lhalf) {
    float bj[FN];  // bias of the lane's column in each block column
#pragma unroll
    for (int b = 0; b < FN; ++b) {
        const int j = j0 + b * 32 + lrow;
        bj[b] = (EPI != kEpiNone && g.bias && j < g.N) ? g.bias[j] : 0.0f;
    }
    // Wait for the bias here, once.  Left to the compiler, the wait lands in
    // every guarded store's branch, and as a full vmcnt(0) (the load may be
    // pending on the path that skipped the previous store), so each store
    // would wait for all earlier ones to complete.
    if (EPI != kEpiNone) __builtin_amdgcn_s_waitcnt(kWaitVm0);
    auto value = [&](float v, int b, float m) {
        if (EPI != kEpiNone) {
            if (g.bias) v = v + bj[b];
            if (g.relu) v = v > 0.0f ? v : 0.0f;
            if (EPI == kEpiAll && g.mask) v = m > 0.0f ? v : 0.0f;
        }
        return v;
    };
#pragma unroll
    for (int a = 0; a < FM; ++a) {
        float mk[FN][16];
        if (EPI == kEpiAll && g.mask) {
#pragma unroll
            for (int b = 0; b < FN; ++b) {
                const int j = j0 + b * 32 + lrow;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int i = i0 + a * 32 + 8 * (r >> 2) + 4 * lhalf + (r & 3);
                    mk[b][r] = (i < g.M && j < g.N) ? g.mask[(size_t)i * g.ldc + j] : 0.0f;
                }
            }
            __builtin_amdgcn_s_waitcnt(kWaitVm0);  // as for the bias
        }
#pragma unroll
        for (int b = 0; b < FN; ++b) {
            const int j = j0 + b * 32 + lrow;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int i = i0 + a * 32 + 8 * (r >> 2) + 4 * lhalf + (r & 3);
                if (i < g.M && j < g.N) Cp[(size_t)i * g.ldc + j] = value(acc[a][b][r], b, mk[b][r]);
            }
        }
        if (EPI == kEpiAll) __builtin_amdgcn_sched_barrier(0);
    }
}

// The epilogue of one element of the split-K sum (store_tile's, elementwise).
__device__ __forceinline__ float epilogue(const GemmArgs &g, float v, int i, int j) {
    if (g.bias) v = v + g.bias[j];
    if (g.relu) v = v > 0.0f ? v : 0.0f;
    if (g.mask) v = g.mask[(size_t)i * g.ldc + j] > 0.0f ? v : 0.0f;
    return v;
}

// Staging of one operand tile: logical [BK][R] (k-major), R = 64, 128 or 256
// rows of the operand's non-k index.  KCONTIG: k is the contiguous index in
// memory (row-major A, or B^T); otherwise the R index is contiguous.
template <int R, int NT, bool KCONTIG>
struct Stage {
    static constexpr int NF = R * kBK / 4 / NT;  // float4 per thread
    static_assert(NF >= 1 && R % 16 == 0, "tile does not divide over the workgroup");

    // float4 number f -> (row, first k) of that float4 in the tile
    static __device__ __forceinline__ void coords(int f, int &row, int &kk) {
        if (KCONTIG) {
            // a wave instruction covers 16 rows x 4 k-quads: 16 lanes per k-quad
            const int grp = f >> 6, l = f & 63;
            const int rb = grp % (R / 16), kb = grp / (R / 16);
            row = rb * 16 + (l & 15);
            kk = 4 * (kb * 4 + (l >> 4));
        } else {
            kk = f / (R / 4);
            row = 4 * (f % (R / 4));
        }
    }

    // a tile with every k inside: one dwordx4 per float4, the row index kept
    // inside the operand (rows past an M / N edge feed outputs that are never
    // stored, so any in-bounds values serve).  Needs the
    // layout of g.vec (16-byte aligned, ld % 4 == 0): for a k-contiguous
    // operand a row is clamped to rows - 1; otherwise a float4 of 4 rows
    // starts at most at (rows - 1) & ~3, which ld >= rows rounded up to 4
    // keeps inside the row.
    static __device__ __forceinline__ void load_clamped(const float *__restrict__ P, int ld, int rows, int r0,
                                                        int k0, f4v_t (&reg)[NF]) {
#pragma unroll
        for (int s = 0; s < NF; ++s) {
            int row, kk;
            coords(s * NT + static_cast<int>(threadIdx.x), row, kk);
            if (KCONTIG) {
                const int r = min(r0 + row, rows - 1);
                reg[s] = *reinterpret_cast<const f4v_t *>(P + (size_t)r * ld + (k0 + kk));
            } else {
                const int r = min(r0 + row, (rows - 1) & ~3);
                reg[s] = *reinterpret_cast<const f4v_t *>(P + (size_t)(k0 + kk) * ld + r);
            }
        }
    }

    // edge tile: element loads with bounds checks, zeros outside
    static __device__ __forceinline__ void load_guarded(const float *__restrict__ P, int ld, int rows,
                                                        int K, int r0, int k0, f4v_t (&reg)[NF]) {
#pragma unroll
        for (int s = 0; s < NF; ++s) {
            int row, kk;
            coords(s * NT + static_cast<int>(threadIdx.x), row, kk);
            float v[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int gr = KCONTIG ? r0 + row : r0 + row + c;
                const int gk = KCONTIG ? k0 + kk + c : k0 + kk;
                v[c] = (gr < rows && gk < K)
                           ? (KCONTIG ? P[(size_t)gr * ld + gk] : P[(size_t)gk * ld + gr])
                           : 0.0f;
            }
            reg[s] = f4v_t{v[0], v[1], v[2], v[3]};
        }
    }

    static __device__ __forceinline__ void store(float *S, const f4v_t (&reg)[NF]) {
#pragma unroll
        for (int s = 0; s < NF; ++s) {
            int row, kk;
            coords(s * NT + static_cast<int>(threadIdx.x), row, kk);
            if (KCONTIG) {
#pragma unroll
                for (int c = 0; c < 4; ++c) S[(kk + c) * R + (row ^ swz(kk + c))] = reg[s][c];
            } else {
                *reinterpret_cast<f4v_t *>(&S[kk * R + (row ^ swz(kk))]) = reg[s];
            }
        }
    }
};

// Tile coordinates of workgroup b of a G-tile grid (see the file comment).
__device__ inline void tile_coords(int tiles_m, int tiles_n, int b, int &tm, int &tn) {
    const int G = tiles_m * tiles_n;
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

// Column sums of B ([K][N], trans_b == 0) for 16 columns, j0 .. j0+15, in
// the column sum's order, by one workgroup of NT threads: in rounds of
// NT/16 chunks, thread (chunk q, column j) adds its chunk's rows from +0 in
// f64 (16 rows in flight at a time, rows past K read in bounds and not
// added), then thread j adds the round's groups of chunk sums, each from +0,
// into its running total, and finally stores it.
constexpr int kStripCols = 16;

template <int NT, bool XF>
__device__ __forceinline__ void colsum_strip(const GemmArgs &g, int j0) {
    constexpr int R = static_cast<int>(kColsumRows), G = static_cast<int>(kColsumGroup), RC = NT / kStripCols;
    static_assert(RC * kStripCols == NT && RC % G == 0, "a round holds whole groups of chunks");
    __shared__ double cs[RC][kStripCols];
    const int t = static_cast<int>(threadIdx.x), q = t / kStripCols, j = t % kStripCols;
    const int col = min(j0 + j, g.N - 1);
    const int chunks = (g.K + R - 1) / R;
    const XfRegs xfb = xf_load(g.xb);
    double total = 0.0;
    for (int c0 = 0; c0 < chunks; c0 += RC) {  // uniform
        const int r0 = (c0 + q) * R;
        double sum = 0.0;
        for (int rb = 0; rb < R; rb += 16) {
            float v[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) v[r] = g.B[(size_t)min(r0 + rb + r, g.K - 1) * g.ldb + col];
            if constexpr (XF) xf_array(xfb, v);  // the rows past K are transformed too, and not added
#pragma unroll
            for (int r = 0; r < 16; ++r)
                if (r0 + rb + r < g.K) sum += (double)v[r];
        }
        cs[q][j] = sum;
        __syncthreads();
        if (t < kStripCols) {
#pragma unroll
            for (int h = 0; h < RC / G; ++h) {
                double grp = 0.0;
#pragma unroll
                for (int i = 0; i < G; ++i) grp += cs[h * G + i][t];
                total += grp;
            }
        }
        __syncthreads();
    }
    if (t < kStripCols && j0 + t < g.N) g.colsum[j0 + t] = static_cast<float>(total);
}

// The sum of GemmArgs::sum_x (sum_n values, each put through sum_xf first,
// one fp32 operation per op as the operand transforms apply them) into
// sum_out[0] with the bits of ts_hip_sum over the transformed values, by one
// workgroup of NT threads (a multiple of kBlock): it plays the sum's
// sum_blocks <= kSumSmallBlocks first-pass workgroups and its second pass.
// Thread T takes the first pass's virtual threads v = T + r*NT (workgroup
// v / kBlock, wave (T % kBlock) / 64, the same lane), each with at most one
// float4 group (and the tail, n - 4*(n/4) < 4 values, on virtual threads
// 0..2), so every wave sum is that pass's; the partials are then combined as
// the second pass combines them (thread t adds partial t from +0, block_sum).
// All loads are issued before any value is used.
template <int NT>
__device__ __forceinline__ void sum_in_workgroup(const GemmArgs &g) {
    static_assert(NT % kBlock == 0, "whole first-pass workgroups per round");
    constexpr int R = kSumSmallBlocks * kBlock / NT;  // rounds
    constexpr int kWaves = kBlock / 64;
    __shared__ double wsum[kSumSmallBlocks][kWaves];
    __shared__ double parts[kSumSmallBlocks];
    __shared__ double fin[kWaves];
    const float *x = g.sum_x;
    const size_t n = g.sum_n, n4 = n / 4;
    const int blocks = g.sum_blocks;
    const int T = static_cast<int>(threadIdx.x), lane = T & 63, wave = T >> 6;
    const XfRegs xs = xf_load(g.sum_xf);
    const size_t ti = 4 * n4 + T < n ? 4 * n4 + T : n - 1;
    float tx[1] = {x[ti]};
    f4v_t q[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        q[r] = f4v_t{0.0f, 0.0f, 0.0f, 0.0f};
        if (r * NT < blocks * kBlock && n4 > 0) {  // uniform
            const size_t v = static_cast<size_t>(T) + static_cast<size_t>(r) * NT;
            q[r] = *reinterpret_cast<const f4v_t *>(x + 4 * (v < n4 ? v : n4 - 1));
        }
    }
    xf_regs(xs, q);
    xf_array(xs, tx);
    double acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        acc[r] = 0.0;
        const size_t v = static_cast<size_t>(T) + static_cast<size_t>(r) * NT;
        if (v < n4) acc[r] += (double)q[r][0] + (double)q[r][1] + (double)q[r][2] + (double)q[r][3];
    }
    if (4 * n4 + T < n) acc[0] += (double)tx[0];
    // every round's butterfly formed together (independent chains), each
    // stored for its first-pass workgroup
    double ws[R];
#pragma unroll
    for (int r = 0; r < R; ++r) ws[r] = wave_sum(acc[r]);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int b = (T + r * NT) / kBlock;
        if (b < blocks && lane == 0) wsum[b][(T % kBlock) / 64] = ws[r];
    }
    __syncthreads();
    if (T < blocks) {
        double s = 0.0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) s += wsum[T][w];
        parts[T] = s;
    }
    __syncthreads();
    if (wave < kWaves) {  // block_sum over the first kBlock threads
        double a = 0.0;
        if (T < blocks) a += parts[T];
        a = wave_sum(a);
        if (lane == 0) fin[wave] = a;
    }
    __syncthreads();
    if (T == 0) {
        double s = 0.0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) s += fin[w];
        const float f = static_cast<float>(s);
        g.sum_out[0] = g.sum_mean ? f / static_cast<float>(n) : f;
    }
}

// EPI: the epilogue kind applied at the store (a separate instantiation per
// kind, so the bare product keeps its register allocation).  PF: operand tiles
// prefetched into registers ahead of the LDS stage (deeper for small tiles,
// whose k-steps are too short to cover a global load).  VEC (operands 16-byte
// aligned, leading dimensions % 4 == 0): the loop runs the whole k tiles with
// dwordx4 loads whose rows are clamped into the operand (rows past an M / N
// edge feed outputs that are never stored), and a partial last tile follows
// it with element loads; otherwise every tile takes bounds-checked element
// loads (zeros outside).  CS (column sums of B): workgroups past the g.tiles
// product tiles each take a strip of kStripCols columns (colsum_strip); the
// grid has no other idle work for them.
template <bool TA, bool TB, int BM, int BN, int WM, int WN, int EPI, int PF, bool VEC, bool CS = false,
          bool XF = false>
__global__ __launch_bounds__(64 * WM * WN) void gemm_f32_mfma(GemmArgs g) {
    static_assert(!CS || !TB, "column sums of B need trans_b == 0");

    if (CS && static_cast<int>(blockIdx.x) >= g.tiles) {  // uniform
        const int j0 = (static_cast<int>(blockIdx.x) - g.tiles) * kStripCols;
        if (j0 < g.N) colsum_strip<64 * WM * WN, XF>(g, j0);
        else sum_in_workgroup<64 * WM * WN>(g);  // the workgroup after the strips: GemmArgs::sum_out
        return;
    }
    constexpr int NT = 64 * WM * WN;
    constexpr int TMW = BM / WM, TNW = BN / WN;  // wave tile
    constexpr int FM = TMW / 32, FN = TNW / 32;  // 32x32 accumulators per wave
    using SA = Stage<BM, NT, !TA>;                // A is k-contiguous unless transposed
    using SB = Stage<BN, NT, TB>;                 // B is k-contiguous only when transposed
    __shared__ __attribute__((aligned(16))) float As[2][kBK * BM];
    __shared__ __attribute__((aligned(16))) float Bs[2][kBK * BN];

    // Batched form: select this workgroup's batch (uniform).  The loop is
    // unrolled with constant indices so the argument arrays stay in SGPRs.
    const float *Ap = g.A, *Bp = g.B;
    float *Cp = g.C;
    int bid = blockIdx.x;
    if (g.batch_rank > 0) {
        const int batch = bid / g.tiles;
        bid -= batch * g.tiles;
        int rem = batch;
        long long oa = 0, ob = 0;
#pragma unroll
        for (int k = kMaxBatchRank - 1; k >= 0; --k) {
            if (k < g.batch_rank) {
                const int c = rem % g.bdims[k];
                rem /= g.bdims[k];
                oa += c * g.sa[k];
                ob += c * g.sb[k];
            }
        }
        Ap += oa;
        Bp += ob;
        Cp += static_cast<long long>(batch) * g.sc;
    }
    int tm, tn;
    tile_coords(g.tiles_m, g.tiles_n, bid, tm, tn);
    const int i0 = tm * BM, j0 = tn * BN;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int lrow = lane & 31, lhalf = lane >> 5;
    const XfRegs xfa = XF ? xf_load(g.xa) : XfRegs{}, xfb = XF ? xf_load(g.xb) : XfRegs{};

    floatx16 acc[FM][FN];
#pragma unroll
    for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;

    // One k tile from LDS: every operand read, then the MFMAs in k order
    // (the reads complete in order, so each MFMA waits only for its own).
    auto mma = [&](const float *Ac, const float *Bc) {
        float af[kBK / 2][FM], bf[kBK / 2][FN];
#pragma unroll
        for (int s = 0; s < kBK / 2; ++s) {
            const int k = 2 * s + lhalf;
#pragma unroll
            for (int a = 0; a < FM; ++a) af[s][a] = Ac[k * BM + ((wm * TMW + a * 32 + lrow) ^ swz(k))];
#pragma unroll
            for (int b = 0; b < FN; ++b) bf[s][b] = Bc[k * BN + ((wn * TNW + b * 32 + lrow) ^ swz(k))];
        }
#pragma unroll
        for (int s = 0; s < kBK / 2; ++s)
#pragma unroll
            for (int a = 0; a < FM; ++a)
#pragma unroll
                for (int b = 0; b < FN; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[s][a], bf[s][b], acc[a][b], 0, 0, 0);
    };

    // Every step issues the same loads (steps past the end re-load the last
    // tile), so the compiler's load counters stay exact and the PF-deep
    // register ring really has PF tiles of loads in flight.
    const int nt = VEC ? g.K / kBK : (g.K + kBK - 1) / kBK;  // tiles of the loop
    f4v_t ra[PF][SA::NF], rb[PF][SB::NF];
    auto load = [&](int t, f4v_t(&a)[SA::NF], f4v_t(&b)[SB::NF]) {
        const int k0 = min(t, nt - 1) * kBK;
        if (VEC) {
            SA::load_clamped(Ap, g.lda, g.M, i0, k0, a);
            SB::load_clamped(Bp, g.ldb, g.N, j0, k0, b);
        } else {
            SA::load_guarded(Ap, g.lda, g.M, g.K, i0, k0, a);
            SB::load_guarded(Bp, g.ldb, g.N, g.K, j0, k0, b);
        }
    };

    if (nt > 0) {
        load(0, ra[0], rb[0]);
        if constexpr (XF) {
            xf_regs(xfa, ra[0]);
            xf_regs(xfb, rb[0]);
        }
        SA::store(As[0], ra[0]);
        SB::store(Bs[0], rb[0]);
#pragma unroll
        for (int p = 0; p < PF; ++p) load(1 + p, ra[p], rb[p]);
        __syncthreads();

        for (int kt0 = 0; kt0 < nt; kt0 += PF) {
#pragma unroll
            for (int u = 0; u < PF; ++u) {
                const int kt = kt0 + u;
                if (kt >= nt) break;  // uniform
                const int cur = kt & 1;
                // LDS[cur] holds tile kt: its operands are read and its MFMAs
                // issued; slot u (tile kt+1, past the end a re-load) goes to
                // buffer cur^1, last read before the previous barrier, and
                // slot u then takes tile kt+1+PF.  One basic block, so the
                // scheduler can place the stores and loads in the MFMAs'
                // shadow (a wave issues in order).
                mma(As[cur], Bs[cur]);
                if constexpr (XF) {
                    xf_regs(xfa, ra[u]);
                    xf_regs(xfb, rb[u]);
                }
                SA::store(As[cur ^ 1], ra[u]);
                SB::store(Bs[cur ^ 1], rb[u]);
                load(kt + 1 + PF, ra[u], rb[u]);
                __syncthreads();
            }
        }
    }
    if (VEC && nt * kBK < g.K) {  // the partial last k tile (uniform)
        f4v_t pa[SA::NF], pb[SB::NF];
        SA::load_guarded(Ap, g.lda, g.M, g.K, i0, nt * kBK, pa);
        SB::load_guarded(Bp, g.ldb, g.N, g.K, j0, nt * kBK, pb);
        if constexpr (XF) {
            xf_regs(xfa, pa);
            xf_regs(xfb, pb);
        }
        SA::store(As[0], pa);
        SB::store(Bs[0], pb);
        __syncthreads();
        mma(As[0], Bs[0]);
    }
    store_tile<EPI, FM, FN>(g, acc, Cp, i0 + wm * TMW, j0 + wn * TNW, lrow, lhalf);
}

// Register prefetch depth per tile size: one tile ahead for 256x256 tiles
// (a k-step of 8 waves' 128x64 blocks is long), four for the smaller ones.
template <int BM>
constexpr int prefetch_tiles() { return BM >= 256 ? 1 : 4; }

template <int BM, int BN, int WM, int WN, int EPI, bool VEC, bool XF>
static void launch_tiles_xf(int ta, int tb, const GemmArgs &g, dim3 grid, dim3 block, hipStream_t s) {
    constexpr int PF = prefetch_tiles<BM>();
    if (g.colsum && ta && !tb) {  // dW with db (no epilogue)
        launch((gemm_f32_mfma<true, false, BM, BN, WM, WN, kEpiNone, PF, VEC, true, XF>), grid, block, 0, s, g);
        return;
    }
    if (!ta && !tb) launch((gemm_f32_mfma<false, false, BM, BN, WM, WN, EPI, PF, VEC, false, XF>), grid, block, 0, s, g);
    else if (!ta && tb) launch((gemm_f32_mfma<false, true, BM, BN, WM, WN, EPI, PF, VEC, false, XF>), grid, block, 0, s, g);
    else if (ta && !tb) launch((gemm_f32_mfma<true, false, BM, BN, WM, WN, EPI, PF, VEC, false, XF>), grid, block, 0, s, g);
    else launch((gemm_f32_mfma<true, true, BM, BN, WM, WN, EPI, PF, VEC, false, XF>), grid, block, 0, s, g);
}

// Operand transforms only on the 64x64 and 128x128 tiles (products with a
// 256x256 grid that fills the chip take none).
template <int BM, int BN, int WM, int WN, int EPI, bool VEC>
static void launch_tiles_vec(int ta, int tb, const GemmArgs &g, dim3 grid, dim3 block, hipStream_t s) {
    if constexpr (BM < 256) {
        if (g.xa.n || g.xb.n) {
            launch_tiles_xf<BM, BN, WM, WN, EPI, VEC, true>(ta, tb, g, grid, block, s);
            return;
        }
    }
    launch_tiles_xf<BM, BN, WM, WN, EPI, VEC, false>(ta, tb, g, grid, block, s);
}

template <int BM, int BN, int WM, int WN, int EPI>
static void launch_tiles_as(int ta, int tb, const GemmArgs &g, dim3 grid, dim3 block, hipStream_t s) {
    if (g.vec) launch_tiles_vec<BM, BN, WM, WN, EPI, true>(ta, tb, g, grid, block, s);
    else launch_tiles_vec<BM, BN, WM, WN, EPI, false>(ta, tb, g, grid, block, s);
}

template <int BM, int BN, int WM, int WN>
static void launch_tiles(int ta, int tb, GemmArgs g, hipStream_t s, unsigned batches = 1) {
    g.tiles_m = (g.M + BM - 1) / BM;
    g.tiles_n = (g.N + BN - 1) / BN;
    g.tiles = g.tiles_m * g.tiles_n;
    dim3 grid(static_cast<unsigned>(g.tiles) * batches);
    // column sums (2-D dW with db): a strip workgroup per 16 columns after the
    // tiles, and one for the sum of B after them
    if (g.colsum && ta && !tb) {
        grid.x += static_cast<unsigned>((g.N + kStripCols - 1) / kStripCols);
        if (g.sum_out) grid.x += 1;
    }
    dim3 block(64 * WM * WN);
    if (g.bias || g.mask || g.relu) launch_tiles_as<BM, BN, WM, WN, kEpiAll>(ta, tb, g, grid, block, s);
    else launch_tiles_as<BM, BN, WM, WN, kEpiNone>(ta, tb, g, grid, block, s);
}

// ---------------------------------------------------------------------------
// LDS-DMA path.  A 256 x 16 operand tile is 1024 16-byte chunks; DMA
// instruction i of wave w carries chunks (NI*w + i)*64 + lane (one 1 KB LDS
// run per instruction: the LDS address is M0 + 16 * lane).
//   KCONTIG: chunk rb*64 + kq*16 + r16 holds row 16*rb + r16, k 4kq .. 4kq+3
//   else:    chunk k*64 + c holds k row k, columns 4*(c ^ dswz(k)) .. +3
// The XOR puts the two k rows one MFMA operand read touches (k and k+2, lane
// halves 0 and 1) in different halves of the bank space.
typedef __attribute__((address_space(3))) void lds_void;
typedef float f2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int dswz(int k) { return ((k >> 1) & 1) << 3; }

template <bool KCONTIG, int NW>
struct DmaStage {
    static constexpr int NI = kBK / NW;  // DMA instructions per wave and operand tile
    static_assert(NI * NW == kBK, "waves must divide the 16 DMA instructions of a tile");

    // DMA instruction i (of NI) of a wave for an interior k tile.  Rows
    // (columns) past the matrix edge are clamped to the last one: they only
    // feed outputs that are never stored.
    static __device__ __forceinline__ void one(const float *__restrict__ P, int ld, int rows, int r0, int k0,
                                               float *S, int wave, int lane, int i) {
        const int q = NI * wave + i;
        const float *src;
        if (KCONTIG) {
            int row = r0 + q * 16 + (lane & 15);
            row = row < rows ? row : rows - 1;
            src = P + (size_t)row * ld + k0 + (lane >> 4) * 4;
        } else {
            const int last = (rows - 1) & ~3;  // ld % 4 == 0, so the chunk stays inside the row
            int col = r0 + 4 * (lane ^ dswz(q));
            col = col <= last ? col : last;
            src = P + (size_t)(k0 + q) * ld + col;
        }
        // Issued as inline assembly: through the builtin the compiler makes
        // every later LDS read wait for this load.  Completion is awaited
        // explicitly (vmcnt) before the barrier that publishes the tile.
        // M0 is listed as clobbered although the compiler treats it as
        // reserved (and warns); nothing else in these kernels uses M0.
        const unsigned lds = static_cast<unsigned>(reinterpret_cast<size_t>((lds_void *)(S + q * 256)));
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds)
                     : "memory", "m0");
#pragma clang diagnostic pop
    }

    // Partial last k tile: element loads with bounds checks, zeros outside.
    static __device__ __forceinline__ void guarded(const float *__restrict__ P, int ld, int rows, int K, int r0,
                                                   int k0, float *S, int wave, int lane) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int q = NI * wave + i;
            float v[4];
            if (KCONTIG) {
                const int row = r0 + q * 16 + (lane & 15), kk = k0 + (lane >> 4) * 4;
#pragma unroll
                for (int c = 0; c < 4; ++c) v[c] = (row < rows && kk + c < K) ? P[(size_t)row * ld + kk + c] : 0.0f;
            } else {
                const int kr = k0 + q, col = r0 + 4 * (lane ^ dswz(q));
#pragma unroll
                for (int c = 0; c < 4; ++c) v[c] = (kr < K && col + c < rows) ? P[(size_t)kr * ld + col + c] : 0.0f;
            }
            *reinterpret_cast<float4 *>(S + q * 256 + lane * 4) = make_float4(v[0], v[1], v[2], v[3]);
        }
    }

    // MFMA operand of steps 2j and 2j+1 for tile-local row (column) rho, lane
    // half h.  An ext_vector pair, not HIP's float2 struct: reads through the
    // struct type make the compiler wait for pending LDS DMA.
    static __device__ __forceinline__ f2v frag(const float *S, int j, int h, int rho) {
        if (KCONTIG) {
            return *reinterpret_cast<const f2v *>(S + (((rho >> 4) * 64 + j * 16 + (rho & 15)) << 2) + 2 * h);
        } else {
            const int k = 4 * j + 2 * h;
            const int o = (((rho >> 2) ^ dswz(k)) << 2) + (rho & 3);
            f2v v;
            v.x = S[k * 256 + o];
            v.y = S[(k + 1) * 256 + o];
            return v;
        }
    }
};

// 256x256 tiles, 2x4 waves (128x64 each, two per SIMD).  A DMA or LDS read
// instruction waits at issue until the CU's address unit or LDS takes it
// (about 16 cycles per 1 KB DMA instruction when one wave issues, 45-60 when
// four do), and a wave issues in order, so with one wave per SIMD each such
// stall idles the matrix core; two waves per SIMD cover each other's.  A step
// pair is 4 groups of 4 MFMAs in (half, a, b) order; its first six MFMAs each
// carry one fragment read of the next pair.  The DMA instructions are spread
// over the MFMAs:
//   SUB 1: three LDS stages of one 16-k tile; k tile kt+2's DMA goes out
//     during k tile kt, one instruction in each step pair's first group, into
//     the buffer k tile kt-1 freed at the last barrier, and is awaited a
//     whole stage later.
//   SUB 2: two stages of two 16-k tiles (half the barriers, for long k);
//     stage kt+1's DMA goes out during the first half of stage kt, two
//     instructions per step pair, into the other buffer, and is awaited at
//     the stage's end (half a stage after the last instruction).
template <bool TA, bool TB, int EPI, bool CS, int SUB>
__global__ __launch_bounds__(512) void gemm_f32_lds_dma(GemmArgs g) {
    constexpr int BM = 256, BN = 256, WM = 2, WN = 4, NW = WM * WN, NB = SUB == 1 ? 3 : 2;
    constexpr int TMW = BM / WM, TNW = BN / WN, FM = TMW / 32, FN = TNW / 32, PAIRS = kBK / 4;
    constexpr int SP = SUB * PAIRS;            // step pairs per stage
    constexpr int NI = kBK / NW, ND = 2 * NI;  // DMA instructions per wave and k tile: A's, then B's
    constexpr int GP = 2 * FM * FN / 4;        // groups of 4 MFMAs per step pair
    static_assert(SUB == 1 || SUB == 2, "one or two k tiles per stage");
    static_assert(FM == 4 && FN == 2 && ND == PAIRS && GP == 4,
                  "DMA slots: one per step pair (SUB 1) or two in each of the first half's (SUB 2)");
    using SA = DmaStage<!TA, NW>;
    using SB = DmaStage<TB, NW>;
    __shared__ __attribute__((aligned(16))) float As[NB][SUB * kBK * BM];
    __shared__ __attribute__((aligned(16))) float Bs[NB][SUB * kBK * BN];

    const float *Ap = g.A, *Bp = g.B;
    float *Cp = g.C;
    int bid = blockIdx.x;
    if (g.batch_rank > 0) {
        const int batch = bid / g.tiles;
        bid -= batch * g.tiles;
        int rem = batch;
        long long oa = 0, ob = 0;
#pragma unroll
        for (int k = kMaxBatchRank - 1; k >= 0; --k) {
            if (k < g.batch_rank) {
                const int c = rem % g.bdims[k];
                rem /= g.bdims[k];
                oa += c * g.sa[k];
                ob += c * g.sb[k];
            }
        }
        Ap += oa;
        Bp += ob;
        Cp += static_cast<long long>(batch) * g.sc;
    }
    int tm, tn;
    tile_coords(g.tiles_m, g.tiles_n, bid, tm, tn);
    const int i0 = tm * BM, j0 = tn * BN;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int lrow = lane & 31, lhalf = lane >> 5;

    floatx16 acc[FM][FN];
#pragma unroll
    for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;

    // CS: the chunk sums of B's columns (GemmArgs::colsum_part) by the first
    // four waves, one column each, from the B tiles in LDS; chunk c (four k
    // tiles) by the workgroups of tile row c % tiles_m.
    static_assert(!CS || !TB, "column sums of B need trans_b == 0");
    const bool cs_wave = CS && wave < 4;  // uniform per wave
    const int cs_c = threadIdx.x & 255;
    double cs_s = 0.0;
    auto cs_mine = [&](int kt) { return ((kt >> 2) % g.tiles_m) == tm; };  // uniform
    auto cs_rows = [&](const float *S, int k0, int k1) {
#pragma unroll
        for (int k = k0; k < k1; ++k) cs_s += (double)S[k * 256 + ((((cs_c >> 2) ^ dswz(k)) << 2) | (cs_c & 3))];
    };
    auto cs_flush = [&](int chunk) {
        if (j0 + cs_c < g.N) g.colsum_part[(size_t)chunk * g.N + j0 + cs_c] = cs_s;
        cs_s = 0.0;
    };
    // the 4 k rows of B of step pair p of stage st (in buffer buf), added
    // before the barrier that frees the buffer; a chunk's fourth k tile closes it
    auto cs_pair = [&](int st, int buf, int p) {
        const int t16 = st * SUB + p / PAIRS, jj = p % PAIRS;
        if (cs_wave && cs_mine(t16)) {
            cs_rows(Bs[buf] + (p / PAIRS) * kBK * BN, 4 * jj, 4 * jj + 4);
            if (jj == PAIRS - 1 && (t16 & 3) == 3) cs_flush(t16 >> 2);
        }
    };

    const int nfull = g.K / (SUB * kBK);  // whole stages; the k tiles past them after the loop
    auto dma1 = [&](int st, int buf, int i) {  // instruction i of stage st: k tile i / ND, A's then B's
        const int s = i / ND, q = i % ND, k0 = (st * SUB + s) * kBK;
        if (q < NI) SA::one(Ap, g.lda, g.M, i0, k0, As[buf] + s * kBK * BM, wave, lane, q);
        else SB::one(Bp, g.ldb, g.N, j0, k0, Bs[buf] + s * kBK * BN, wave, lane, q - NI);
    };
    f2v F[2][FM + FN];
    auto rd1 = [&](int buf, int j, f2v (&f)[FM + FN], int k) {  // fragment k of step pair j of a stage
        const float *Sa = As[buf] + (j / PAIRS) * kBK * BM, *Sb = Bs[buf] + (j / PAIRS) * kBK * BN;
        if (k < FM) f[k] = SA::frag(Sa, j % PAIRS, lhalf, wm * TMW + k * 32 + lrow);
        else f[k] = SB::frag(Sb, j % PAIRS, lhalf, wn * TNW + (k - FM) * 32 + lrow);
    };
    auto mfma = [&](const f2v (&f)[FM + FN], int idx) {  // MFMA idx of a step pair, (half, a, b) order
        const int h = idx / (FM * FN), a = (idx / FN) % FM, b = idx % FN;
        acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(h ? f[a].y : f[a].x, h ? f[FM + b].y : f[FM + b].x,
                                                         acc[a][b], 0, 0, 0);
    };
    // Step pair p of the current stage from registers f; fragments of step
    // pair jn of buffer rb into n; this pair's DMA instructions of stage ks
    // into dst.
    auto pair = [&](const f2v (&f)[FM + FN], f2v (&n)[FM + FN], int rb, int jn, int p, int ks, int dst) {
#pragma unroll
        for (int grp = 0; grp < GP; ++grp) {
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                mfma(f, grp * 4 + m);
                if (grp * 4 + m < FM + FN) rd1(rb, jn, n, grp * 4 + m);
            }
            if (grp == 0) {
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
                }
            } else if (grp == 1) {
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    if (4 + m < FM + FN) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            if (SUB == 1 && grp == 0) dma1(ks, dst, p);
            if (SUB == 2 && p < PAIRS && (grp == 0 || grp == 2)) dma1(ks, dst, 2 * p + grp / 2);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Pipeline (SUB 1): buffer kt % 3 holds k tile kt; k tile kt+1 has landed
    // or is landing in the next; k tile kt+2 is loaded into the third during
    // this one (its buffer held kt-1, whose reads all precede the last
    // barrier).  Each wave waits for its own DMA (vmcnt; loads complete in
    // order) before the barrier that publishes a stage: of the 2*ND
    // instructions in flight there, the last ND-1 are k tile kt+2's.
    // (SUB 2): buffer kt & 1 holds stage kt, stage kt+1 is loaded into the
    // other during its first half, and all of it is awaited (vmcnt(0)).
    if (nfull > 0) {
#pragma unroll
        for (int i = 0; i < SUB * ND; ++i) dma1(0, 0, i);
        if (SUB == 1) {
#pragma unroll
            for (int i = 0; i < ND; ++i) dma1(nfull > 1 ? 1 : 0, 1, i);
            asm volatile("s_waitcnt vmcnt(4)" ::: "memory");  // ND: k tile 0 has landed
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < FM + FN; ++k) rd1(0, 0, F[0], k);
    }
    int cur = 0;
    for (int kt = 0; kt < nfull; ++kt) {
        const int nxt = cur == NB - 1 ? 0 : cur + 1;
        const int dst = SUB == 1 ? (nxt == NB - 1 ? 0 : nxt + 1) : nxt;
        // past the end the DMA repeats the last stage into the free buffer
        // and the last read takes it: both stay in bounds, neither is used
        const int ahead = kt + (SUB == 1 ? 2 : 1);
        const int ks = ahead < nfull ? ahead : nfull - 1;
#pragma unroll
        for (int j = 0; j < SP - 1; ++j) {
            pair(F[j & 1], F[(j + 1) & 1], cur, j + 1, j, ks, dst);
            if (CS) {
                cs_pair(kt, cur, j);
                if (j == SP - 2) cs_pair(kt, cur, j + 1);
            }
        }
        if (SUB == 1) asm volatile("s_waitcnt vmcnt(3)" ::: "memory");  // ND - 1
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        pair(F[(SP - 1) & 1], F[0], nxt, 0, SP - 1, ks, dst);
        cur = nxt;
    }
    // the k tiles past the last whole stage (the last may be partial), one at
    // a time with bounds checks through buffer 0 (idle: every DMA has landed
    // and every read passed the barrier)
    for (int t16 = nfull * SUB; t16 * kBK < g.K; ++t16) {  // uniform
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        SA::guarded(Ap, g.lda, g.M, g.K, i0, t16 * kBK, As[0], wave, lane);
        SB::guarded(Bp, g.ldb, g.N, g.K, j0, t16 * kBK, Bs[0], wave, lane);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < PAIRS; ++j) {
#pragma unroll
            for (int k = 0; k < FM + FN; ++k) rd1(0, j, F[0], k);
#pragma unroll
            for (int m = 0; m < 2 * FM * FN; ++m) mfma(F[0], m);
        }
        if (cs_wave && cs_mine(t16)) {  // zeros past K add nothing
            cs_rows(Bs[0], 0, kBK);
            if ((t16 & 3) == 3) cs_flush(t16 >> 2);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no DMA outstanding at exit
    if (CS) {  // the last chunk, unless its fourth k tile closed it
        const int last = (g.K - 1) / kBK;
        if (cs_wave && cs_mine(last) && (last & 3) != 3) cs_flush(last >> 2);
    }

    store_tile<EPI, FM, FN>(g, acc, Cp, i0 + wm * TMW, j0 + wn * TNW, lrow, lhalf);
}

// Split-K: C[i][j] = sum over s of the slice products P_s[i][j] (P_s at
// P + s*M*N, row-major M x N), added in slice order; at most 16 slices (both
// splitting paths stay within that).
__global__ __launch_bounds__(kBlock) void splitk_sum(const float *__restrict__ P, int slices, size_t M, size_t N,
                                                     float *__restrict__ C, size_t ldc, GemmArgs e) {
    const size_t t = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
    const size_t mn = M * N;
    if (e.colsum && blockIdx.x == gridDim.x - 1) {
        // The skinny product's column sums of B (N <= 16), in the column sum's
        // order, by the workgroup past the product: in rounds of 16 chunks,
        // thread (chunk lane q, column j) adds its chunk's rows (all loaded at
        // once), then the first lane adds the round's two groups of chunk sums
        // in order.
        constexpr int R = static_cast<int>(kColsumRows), G = static_cast<int>(kColsumGroup);
        __shared__ double cs[16][17];
        const int j = threadIdx.x & 15, q = threadIdx.x >> 4;
        const size_t chunks = colsum_chunk_count(static_cast<size_t>(e.K));
        double total = 0.0;
        for (size_t c0 = 0; c0 < chunks; c0 += 16) {  // uniform
            const size_t c = c0 + q;
            double sum = 0.0;
            if (j < e.N && c < chunks) {
                float v[R];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const size_t k = c * R + r;
                    v[r] = k < static_cast<size_t>(e.K) ? e.B[k * e.ldb + j] : 0.0f;
                }
#pragma unroll
                for (int r = 0; r < R; ++r) sum += (double)v[r];
            }
            cs[q][j] = sum;
            __syncthreads();
            if (q == 0) {
#pragma unroll
                for (int h = 0; h < 16 / G; ++h) {
                    double grp = 0.0;
#pragma unroll
                    for (int i = 0; i < G; ++i) grp += cs[h * G + i][j];
                    total += grp;
                }
            }
            __syncthreads();
        }
        if (q == 0 && j < e.N) e.colsum[j] = static_cast<float>(total);
        return;
    }
    if (t >= mn) return;
    // every slice's value in flight at once (slices <= 16), then the sum in slice order
    float v[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = k < slices ? P[static_cast<size_t>(k) * mn + t] : 0.0f;
    float acc = v[0];
#pragma unroll
    for (int k = 1; k < 16; ++k)
        if (k < slices) acc += v[k];
    const size_t i = t / N, j = t % N;
    C[i * ldc + j] = epilogue(e, acc, static_cast<int>(i), static_cast<int>(j));
}

// ---------------------------------------------------------------------------
// 16x16x4 path for exact tilings (M and N multiples of 256, K of 32, no batch
// rank): 256x256 tiles, 8 waves of 128x64, each 8x4 blocks of
// v_mfma_f32_16x16x4_f32, two LDS stages of 32 k rows fed by LDS DMA.
//
// Every operand read is a 16-byte ds_read_b128 that feeds four MFMAs:
//   k-major operand (stored [K][rows]): LDS stage [k][256]; lane (i, q) reads
//     the 4 consecutive rows (columns) 64g + 4i .. +3 at k row kk, the operand
//     of blocks 4g + 0 .. 4g + 3 (block b's lane i is row 64g + 4i + b);
//   k-contiguous operand (stored [rows][K]): 16-byte chunks of 4 k, chunk
//     (rho >> 4) * 128 + kq * 16 + (rho & 15) for LDS row rho and k quad kq,
//     and LDS row rho holds matrix row w16_perm(rho) (the same interleave:
//     block 4g + b's lane i is row 64g + 4i + b); lane (i, q) reads 4 k of
//     one block, its operand for 4 k steps.
// K step ks of a stage takes, in lane group q, k row 16 (ks / 4) + 4q + ks % 4
// (the k-contiguous reads fix that order; the k-major reads follow it), so a
// block's 16 k of a super step are added in another order than the 32x32
// kernels' (a different rounding of the same sum).  A lane's accumulator
// element v of blocks (4g + b, c) is C[64g + 16q + 4v + b][4i + c]: four
// adjacent columns, stored as one 16-byte store.
//
// The DMA uses the scalar-base form (a wave-uniform row base in SGPRs plus a
// 32-bit lane offset shared by all of a wave's instructions of one operand):
// with a 64-bit address per instruction the compiler kept all eight live
// across the loop and spilled.  The stage barrier comes before a stage's last
// k step (vmcnt and lgkmcnt at zero first: the next stage has landed, and
// every read of this buffer is done), so that k step's MFMAs cover the first
// reads of the next stage.  SCHED picks where a stage's 8 DMA instructions go:
// 0 two per k step over the first four, 1 one per k step over the first six
// and two more in the first two.
constexpr int kW16K = 32;
__device__ __forceinline__ int w16_perm(int r) { return (r & ~63) | (4 * (r & 15) + ((r >> 4) & 3)); }

template <bool KC>
struct W16Op {
    static __device__ __forceinline__ unsigned lane_off(int ld, int lane) {
        return KC ? static_cast<unsigned>((4 * (lane & 15) * ld + 4 * (lane >> 4)) * 4)
                  : static_cast<unsigned>(16 * lane);
    }
    // DMA instruction r (0..31) of the stage at k0 into S
    static __device__ __forceinline__ void dma(const float *__restrict__ P, int ld, int r0, int k0, float *S, int r,
                                               unsigned voff) {
        const float *base;
        float *dst;
        if (KC) {
            const int rb = r >> 1, hh = r & 1;
            base = P + (size_t)(r0 + 64 * (rb >> 2) + (rb & 3)) * ld + k0 + 16 * hh;
            dst = S + (rb * 128 + hh * 64) * 4;
        } else {
            base = P + (size_t)(k0 + r) * ld + r0;
            dst = S + r * 256;
        }
        const unsigned lds = static_cast<unsigned>(reinterpret_cast<size_t>((lds_void *)dst));
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
        asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(lds)
                     : "memory", "m0");
#pragma clang diagnostic pop
    }
    // k-contiguous: block x (LDS rows base + 16x .., base a multiple of 16)
    // for super step sg: chunk ((base >> 4) + x) * 128 + (4 sg + q) * 16 + i,
    // i.e. the lane index times 4 floats past a wave-uniform offset (written
    // so: from the chunk formula the compiler kept an address per block,
    // super step and buffer)
    static __device__ __forceinline__ f4v_t kc(const float *S, int base, int x, int sg, int lane) {
        return *reinterpret_cast<const f4v_t *>(S + ((base >> 4) + x) * 512 + sg * 256 + lane * 4);
    }
    // k-major: group gi (blocks 4gi .. 4gi+3) at k row kk
    static __device__ __forceinline__ f4v_t km(const float *S, int base, int gi, int kk, int li) {
        return *reinterpret_cast<const f4v_t *>(S + kk * 256 + base + 64 * gi + 4 * li);
    }
};

// CS (TN only): B's column chunk sums as gemm_f32_lds_dma forms them (chunk c
// of 64 k rows by the workgroups of tile row c % tiles_m, each column's rows
// added in order from +0 in f64) by the first four waves from the B stages
// in LDS: a stage's 32 rows over its first six k steps (5, 5, 5, 5, 6, 6),
// each k step's rows read at its 5th MFMA and added at its 21st (read and
// added at once, the waits for the reads made those four waves late at every
// barrier: 22 us per 4096x4096x8192 product, against 6 us so).
template <bool TA, bool TB, int EPI, bool CS, int SCHED>
__global__ __launch_bounds__(512) void gemm_f32_w16(GemmArgs g) {
    constexpr bool KCA = !TA, KCB = TB;
    static_assert(!CS || (TA && !TB), "column sums on the TN layout only");
    __shared__ __attribute__((aligned(16))) float As[2][kW16K * 256];
    __shared__ __attribute__((aligned(16))) float Bs[2][kW16K * 256];
    int tm, tn;
    tile_coords(g.tiles_m, g.tiles_n, blockIdx.x, tm, tn);
    const int i0 = tm * 256, j0 = tn * 256;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave >> 2, wn = wave & 3;
    const int li = lane & 15, lq = lane >> 4;
    const int abase = wm * 128, bbase = wn * 64;
    f4v_t acc[8][4];
#pragma unroll
    for (int a = 0; a < 8; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = f4v_t{0.0f, 0.0f, 0.0f, 0.0f};

    const bool cs_wave = CS && wave < 4;  // uniform
    const int cs_c = threadIdx.x & 255;
    double cs_s = 0.0;
    float cs_v[6];
    auto cs_first = [](int ks) { return ks < 4 ? 5 * ks : 20 + 6 * (ks - 4); };
    auto cs_count = [](int ks) { return ks < 4 ? 5 : 6; };
    auto cs_load = [&](int buf, int st, int ks) {
        if (cs_wave && ((st >> 1) % g.tiles_m) == tm)
#pragma unroll
            for (int r = 0; r < cs_count(ks); ++r) cs_v[r] = Bs[buf][(cs_first(ks) + r) * 256 + cs_c];
    };
    auto cs_add = [&](int st, int ks) {
        if (cs_wave && ((st >> 1) % g.tiles_m) == tm)
#pragma unroll
            for (int r = 0; r < cs_count(ks); ++r) cs_s += (double)cs_v[r];
    };
    auto cs_flush = [&](int st) {
        if (cs_wave && ((st >> 1) % g.tiles_m) == tm) {
            g.colsum_part[(size_t)(st >> 1) * g.N + j0 + cs_c] = cs_s;
            cs_s = 0.0;
        }
    };

    const unsigned voff = wave < 4 ? W16Op<KCA>::lane_off(g.lda, lane) : W16Op<KCB>::lane_off(g.ldb, lane);
    auto dma = [&](int st, int buf, int i) {  // instruction i (0..7) of this wave: A's 32, then B's
        const int r = wave * 8 + i;
        if (r < 32) W16Op<KCA>::dma(g.A, g.lda, i0, st * kW16K, As[buf], r, voff);
        else W16Op<KCB>::dma(g.B, g.ldb, j0, st * kW16K, Bs[buf], r - 32, voff);
    };
    f4v_t FAm[2][2], FAc[8], FBm[2], FBc[2][4];
    auto kk_of = [&](int ks) { return 16 * (ks >> 2) + 4 * lq + (ks & 3); };
    auto rd_km = [&](int buf, int ks, int slot) {
        if (!KCA) {
            FAm[slot][0] = W16Op<false>::km(As[buf], abase, 0, kk_of(ks), li);
            FAm[slot][1] = W16Op<false>::km(As[buf], abase, 1, kk_of(ks), li);
        }
        if (!KCB) FBm[slot] = W16Op<false>::km(Bs[buf], bbase, 0, kk_of(ks), li);
    };
    auto rd_kcb = [&](int buf, int sg, int slot) {
        if (KCB)
#pragma unroll
            for (int c = 0; c < 4; ++c) FBc[slot][c] = W16Op<true>::kc(Bs[buf], bbase, c, sg, lane);
    };
    auto rd_kca = [&](int buf, int sg, int x) {
        if (KCA) FAc[x] = W16Op<true>::kc(As[buf], abase, x, sg, lane);
    };
    auto mf = [&](int ks, int idx) {  // A block x = idx / 4, B block c = idx % 4
        const int x = idx >> 2, c = idx & 3, s = ks & 3, slot = ks & 1, bslot = (ks >> 2) & 1;
        const float a = KCA ? FAc[x][s] : FAm[slot][x >> 2][x & 3];
        const float b = KCB ? FBc[bslot][c][s] : FBm[slot][c];
        acc[x][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[x][c], 0, 0, 0);
    };

    const int nst = g.K / kW16K;  // >= 1
#pragma unroll
    for (int i = 0; i < 8; ++i) dma(0, 0, i);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    rd_km(0, 0, 0);
    rd_kcb(0, 0, 0);
#pragma unroll
    for (int x = 0; x < 8; ++x) rd_kca(0, 0, x);
    for (int st = 0; st < nst; ++st) {
        const int buf = st & 1, nb = buf ^ 1;
        // past the last stage the DMA reloads it into the free buffer (in bounds, never read)
        const int sn = st + 1 < nst ? st + 1 : st;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            if (ks == 7) {
                asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
                __syncthreads();
            }
            const int rbuf = ks == 7 ? nb : buf;  // the reads issued in this k step: the next one's
#pragma unroll
            for (int idx = 0; idx < 32; ++idx) {
                mf(ks, idx);
                if (idx == 1) rd_km(rbuf, (ks + 1) & 7, (ks + 1) & 1);
                if (KCB && (ks & 3) == 3 && idx == 3) rd_kcb(rbuf, ((ks + 1) >> 2) & 1, ((ks >> 2) + 1) & 1);
                if (KCA && (ks & 3) == 3 && (idx & 3) == 3) rd_kca(rbuf, ((ks + 1) >> 2) & 1, idx >> 2);
                if (SCHED == 1) {
                    if (ks < 6 && idx == 16) dma(sn, nb, ks);
                    if (ks < 2 && idx == 24) dma(sn, nb, 6 + ks);
                } else {
                    if (ks < 4 && (idx == 8 || idx == 24)) dma(sn, nb, 2 * ks + (idx >> 4));
                }
                if (CS && idx == 4 && ks < 6) cs_load(buf, st, ks);
                if (CS && idx == 20 && ks < 6) cs_add(st, ks);
                __builtin_amdgcn_sched_barrier(0);  // reads and DMA stay where they are written
            }
        }
        if (CS && (st & 1)) cs_flush(st);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no DMA outstanding at exit
    if (CS && (nst & 1)) cs_flush(nst - 1);            // a last chunk of one stage

    // store, with the epilogue of store_tile (bias, relu, then the mask); the
    // bias loaded once and each row group's 16 mask vectors before its first
    // store, each batch awaited once (each vector loaded just before its
    // store, every load's latency was waited out in turn)
    float *Cp = g.C;
    const bool vec = ((reinterpret_cast<uintptr_t>(Cp) & 15) == 0) && (g.ldc % 4 == 0) &&
                     (EPI != kEpiAll || !g.mask || (reinterpret_cast<uintptr_t>(g.mask) & 15) == 0);
    const int col = j0 + bbase + 4 * li;
    float bj[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (EPI != kEpiNone && g.bias) {
#pragma unroll
        for (int c = 0; c < 4; ++c) bj[c] = g.bias[col + c];
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
    }
#pragma unroll
    for (int gg = 0; gg < 2; ++gg) {
        f4v_t mk[4][4];
        if (EPI == kEpiAll && g.mask) {
#pragma unroll
            for (int v = 0; v < 4; ++v)
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const size_t at = (size_t)(i0 + abase + 64 * gg + 16 * lq + 4 * v + b) * g.ldc + col;
                    if (vec) {
                        mk[v][b] = *reinterpret_cast<const f4v_t *>(g.mask + at);
                    } else {
#pragma unroll
                        for (int c = 0; c < 4; ++c) mk[v][b][c] = g.mask[at + c];
                    }
                }
            __builtin_amdgcn_s_waitcnt(kWaitVm0);
        }
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int x = 4 * gg + b;
                const size_t at = (size_t)(i0 + abase + 64 * gg + 16 * lq + 4 * v + b) * g.ldc + col;
                float o[4] = {acc[x][0][v], acc[x][1][v], acc[x][2][v], acc[x][3][v]};
                if (EPI != kEpiNone) {
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        float val = o[c];
                        if (g.bias) val = val + bj[c];
                        if (g.relu) val = val > 0.0f ? val : 0.0f;
                        if (EPI == kEpiAll && g.mask) val = mk[v][b][c] > 0.0f ? val : 0.0f;
                        o[c] = val;
                    }
                }
                if (vec) {
                    *reinterpret_cast<f4v_t *>(Cp + at) = f4v_t{o[0], o[1], o[2], o[3]};
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c) Cp[at + c] = o[c];
                }
            }
        if (EPI == kEpiAll) __builtin_amdgcn_sched_barrier(0);
    }
}

template <bool TA, bool TB, int EPI, bool CS, int SCHED>
static void launch_w16(GemmArgs g, hipStream_t s) {
    g.tiles_m = g.M / 256;
    g.tiles_n = g.N / 256;
    g.tiles = g.tiles_m * g.tiles_n;
    launch((gemm_f32_w16<TA, TB, EPI, CS, SCHED>), dim3(static_cast<unsigned>(g.tiles)), dim3(512), 0, s, g);
}

// The 16x16x4 kernel takes a product when its tiling is exact, it has no
// batch rank and the lane offsets of its DMA fit 32 bits.
static bool w16_fits(const GemmArgs &g, unsigned batches) {
    const long long lim = 1LL << 31;
    return batches == 1 && g.batch_rank == 0 && g.M % 256 == 0 && g.N % 256 == 0 && g.K % kW16K == 0 &&
           g.K >= kW16K && 64LL * g.lda * 4 < lim && 64LL * g.ldb * 4 < lim;
}

template <bool TA, bool TB, int EPI, bool CS = false, int SUB = 1>
static void launch_dma(GemmArgs g, hipStream_t s, unsigned batches) {
    g.tiles_m = (g.M + 255) / 256;
    g.tiles_n = (g.N + 255) / 256;
    g.tiles = g.tiles_m * g.tiles_n;
    dim3 grid(static_cast<unsigned>(g.tiles) * batches);
    dim3 block(512);
    launch((gemm_f32_lds_dma<TA, TB, EPI, CS, SUB>), grid, block, 0, s, g);
}

// The DMA kernel of one layout and epilogue (only these instantiations exist):
// two k tiles per stage for TN, whose k is the batch (long), one otherwise,
// the faster measured per layout.
static void launch_dma_layout(int ta, int tb, const GemmArgs &g, hipStream_t s, unsigned nb) {
    const bool epi = g.bias || g.mask || g.relu;
    // the 16x16x4 kernel for NN, NT and TN (its DMA spread measured per
    // layout; NT alone ran as fast on either kernel, in config 5's step 44 us
    // faster per launch on this one)
    if (!(ta && tb) && w16_fits(g, nb)) {
        if (!ta && tb) {
            if (epi) launch_w16<false, true, kEpiAll, false, 0>(g, s);
            else launch_w16<false, true, kEpiNone, false, 0>(g, s);
        } else if (!ta) {
            if (g.mask) launch_w16<false, false, kEpiAll, false, 1>(g, s);
            else if (epi) launch_w16<false, false, kEpiBiasRelu, false, 1>(g, s);
            else launch_w16<false, false, kEpiNone, false, 1>(g, s);
        } else {
            if (g.colsum) launch_w16<true, false, kEpiNone, true, 0>(g, s);
            else if (epi) launch_w16<true, false, kEpiAll, false, 0>(g, s);
            else launch_w16<true, false, kEpiNone, false, 0>(g, s);
        }
        return;
    }
    if (!ta && !tb) {
        if (g.mask) launch_dma<false, false, kEpiAll>(g, s, nb);
        else if (epi) launch_dma<false, false, kEpiBiasRelu>(g, s, nb);
        else launch_dma<false, false, kEpiNone>(g, s, nb);
    } else if (!ta && tb) {
        if (epi) launch_dma<false, true, kEpiAll>(g, s, nb);
        else launch_dma<false, true, kEpiNone>(g, s, nb);
    } else if (ta && !tb) {
        if (g.colsum) launch_dma<true, false, kEpiNone, true, 2>(g, s, nb);  // dW with db
        else if (epi) launch_dma<true, false, kEpiAll, false, 2>(g, s, nb);
        else launch_dma<true, false, kEpiNone, false, 2>(g, s, nb);
    } else {
        if (epi) launch_dma<true, true, kEpiAll>(g, s, nb);
        else launch_dma<true, true, kEpiNone>(g, s, nb);
    }
}

// ---- launch groups -------------------------------------------------------------
//
// Between ts_hip_launch_group_begin(stream) and ts_hip_launch_group_end(stream)
// the calling thread's products on that stream that run on the narrow or the
// one-k-tile kernel are held (at most two); any other launch on the stream
// launches them first, in the order they were issued.  At the end, one of each
// runs as one launch when their pair is instantiated (gemm_narrow_short_k: an
// MLP backward's dW with its bias gradient and dX of a layer with few outputs,
// both latency-bound), otherwise what is held is launched as issued.
namespace {
enum : int { kHeldNarrow = 1, kHeldShortK = 2 };
struct HeldLaunch {
    int kind, variant;
    void (*kernel)(GemmArgs);
    dim3 grid, block;
    GemmArgs g;
};
struct LaunchGroupState {
    bool open = false;
    hipStream_t stream = nullptr;
    int n = 0;
    HeldLaunch held[2];
};
thread_local LaunchGroupState t_group;

// held when a group is open on s with room, else launched (after any held)
void hold_or_launch(int kind, int variant, void (*k)(GemmArgs), dim3 grid, dim3 block, hipStream_t s,
                    const GemmArgs &g) {
    LaunchGroupState &lg = t_group;
    if (lg.open && lg.stream == s && lg.n < 2) {
        lg.held[lg.n++] = HeldLaunch{kind, variant, k, grid, block, g};
        return;
    }
    launch(k, grid, block, 0, s, g);
}
}  // namespace

bool launch_group_holding() { return t_group.n > 0; }

void flush_launch_group() {
    LaunchGroupState &lg = t_group;
    const int n = lg.n;
    lg.n = 0;
    for (int i = 0; i < n; ++i) launch_now(lg.held[i].kernel, lg.held[i].grid, lg.held[i].block, 0, lg.stream, lg.held[i].g);
}

template <bool TA, bool TB, bool V, bool CS, bool XF>
constexpr int narrow_variant() {
    return int(TA) | int(TB) << 1 | int(V) << 2 | int(CS) << 3 | int(XF) << 4;
}
template <bool TA, bool TB, int EPI, bool XF>
constexpr int short_k_variant() {
    return int(TA) | int(TB) << 1 | EPI << 2 | int(XF) << 4;
}

// ---- short contractions (K <= 16) --------------------------------------------
//
// One k tile: a wave's 32x32 block takes at most 8 MFMAs, so its operands go
// from global memory straight to registers (no LDS, no barrier), and the
// epilogue's mask and bias are loaded beside them rather than after the
// MFMAs: one round of loads, the MFMAs, the stores.  64x64 workgroup tiles
// of four 32x32 waves, numbered as the tiled kernels number theirs; MFMA s
// takes k = 2s + (lane half), as a tiled kernel's k tile does, and stops at
// the last MFMA that holds a k < K (the tiled kernels add the zero products
// of the rest), so the stored values are the same.
// Tile `tile` of the grid, by the 256 threads numbered tid (4 waves).
template <bool TA, bool TB, int EPI, bool XF>
__device__ __forceinline__ void short_k_tile(const GemmArgs &g, int tile, int tid) {
    int tm, tn;
    tile_coords(g.tiles_m, g.tiles_n, tile, tm, tn);
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lrow = lane & 31, lhalf = lane >> 5;
    const int i0 = tm * 64 + (wave >> 1) * 32, j = tn * 64 + (wave & 1) * 32 + lrow;
    const float *__restrict__ A = g.A;
    const float *__restrict__ B = g.B;
    // Every load is unconditional, at an in-bounds address (rows and columns
    // past the edge read the last one and feed outputs that are never
    // stored; k past K reads k = K-1 and is replaced by zero), so all of
    // them are in flight together: a load under a condition makes the
    // compiler wait for it before the next.
    // The operands are issued first: the mask values are consumed early (as
    // compare results), which waits for every load issued before them.
    const int ia = min(i0 + lrow, g.M - 1), jb = min(j, g.N - 1);
    float af[kBK / 2], bf[kBK / 2];
#pragma unroll
    for (int s = 0; s < kBK / 2; ++s) {
        const int k = min(2 * s + lhalf, g.K - 1);
        const float a = TA ? A[(size_t)k * g.lda + ia] : A[(size_t)ia * g.lda + k];
        const float b = TB ? B[(size_t)jb * g.ldb + k] : B[(size_t)k * g.ldb + jb];
        const bool in = 2 * s + lhalf < g.K;
        af[s] = in ? a : 0.0f;
        bf[s] = in ? b : 0.0f;
    }
    float mk[16], bj = 0.0f;
    if (EPI != kEpiNone) {
        if (g.bias) bj = g.bias[jb];  // uniform
        if (EPI == kEpiAll && g.mask) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int i = min(i0 + 8 * (r >> 2) + 4 * lhalf + (r & 3), g.M - 1);
                mk[r] = g.mask[(size_t)i * g.ldc + jb];
            }
        }
    }
    if constexpr (XF) {  // after the mask loads are issued: transforming waits for the operands
        xf_array(xf_load(g.xa), af);
        xf_array(xf_load(g.xb), bf);
    }
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    const int steps = (g.K + 1) / 2;  // uniform
#pragma unroll
    for (int s = 0; s < kBK / 2; ++s)
        if (s < steps) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(af[s], bf[s], acc, 0, 0, 0);
    if (j >= g.N) return;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int i = i0 + 8 * (r >> 2) + 4 * lhalf + (r & 3);
        float v = acc[r];
        if (EPI != kEpiNone) {  // store_tile's order: bias, relu, mask
            if (g.bias) v = v + bj;
            if (g.relu) v = v > 0.0f ? v : 0.0f;
            if (EPI == kEpiAll && g.mask) v = mk[r] > 0.0f ? v : 0.0f;
        }
        if (i < g.M) g.C[(size_t)i * g.ldc + j] = v;
    }
}

template <bool TA, bool TB, int EPI, bool XF = false>
__global__ __launch_bounds__(256) void gemm_short_k(GemmArgs g) {
    short_k_tile<TA, TB, EPI, XF>(g, blockIdx.x, threadIdx.x);
}

template <bool TA, bool TB, int EPI, bool XF>
static void short_k_launch(dim3 grid, hipStream_t s, const GemmArgs &g) {
    hold_or_launch(kHeldShortK, short_k_variant<TA, TB, EPI, XF>(), gemm_short_k<TA, TB, EPI, XF>, grid, dim3(256), s,
                   g);
}

template <int EPI, bool XF>
static void launch_short_k_xf(int ta, int tb, const GemmArgs &g, dim3 grid, hipStream_t s) {
    if (!ta && !tb) short_k_launch<false, false, EPI, XF>(grid, s, g);
    else if (!ta) short_k_launch<false, true, EPI, XF>(grid, s, g);
    else if (!tb) short_k_launch<true, false, EPI, XF>(grid, s, g);
    else short_k_launch<true, true, EPI, XF>(grid, s, g);
}

template <int EPI>
static void launch_short_k_as(int ta, int tb, const GemmArgs &g, dim3 grid, hipStream_t s) {
    if (g.xa.n || g.xb.n) launch_short_k_xf<EPI, true>(ta, tb, g, grid, s);
    else launch_short_k_xf<EPI, false>(ta, tb, g, grid, s);
}

static void launch_short_k(int ta, int tb, GemmArgs g, hipStream_t s) {
    g.tiles_m = (g.M + 63) / 64;
    g.tiles_n = (g.N + 63) / 64;
    g.tiles = g.tiles_m * g.tiles_n;
    const dim3 grid(static_cast<unsigned>(g.tiles));
    if (g.bias || g.mask || g.relu) launch_short_k_as<kEpiAll>(ta, tb, g, grid, s);
    else launch_short_k_as<kEpiNone>(ta, tb, g, grid, s);
}

}  // namespace tship

using namespace tship;

// Enough 256x256 tiles to fill every CU: the LDS-DMA kernel when the operands
// allow dwordx4 loads (vec), else 256x256 register-staged tiles.
static bool big_grid(size_t M, size_t N, size_t batches) {
    return ((M + 255) / 256) * ((N + 255) / 256) * batches >= static_cast<size_t>(device_cu_count());
}

static bool vec_operands(const float *A, size_t lda, const float *B, size_t ldb) {
    return aligned16(A) && aligned16(B) && (lda % 4 == 0) && (ldb % 4 == 0);
}

// Argument checks and kernel selection shared by the plain and batched forms.
static int gemm_launch(int trans_a, int trans_b, size_t M, size_t N, size_t K, const float *A, size_t lda,
                       const float *B, size_t ldb, float *C, size_t ldc, GemmArgs g, size_t batches,
                       void *stream) {
    if (!A || !B) return TS_HIP_EINVAL;
    if (lda < (trans_a ? M : K) || ldb < (trans_b ? K : N)) return TS_HIP_EINVAL;
    // dimensions and leading dimensions are 32-bit inside the kernel (element
    // offsets are formed in 64 bits), and the workgroup count must fit one grid
    const size_t lim = 0x7ffffe00ULL;  // room for i0 + BM within int
    if (M > lim || N > lim || K > lim || lda > lim || ldb > lim || ldc > lim) return TS_HIP_EINVAL;
    if (((M + 127) / 128) * ((N + 127) / 128) * batches > 0x7fffffffULL) return TS_HIP_EINVAL;
    g.A = A; g.B = B; g.C = C;
    g.M = static_cast<int>(M); g.N = static_cast<int>(N); g.K = static_cast<int>(K);
    g.lda = static_cast<int>(lda); g.ldb = static_cast<int>(ldb); g.ldc = static_cast<int>(ldc);
    g.tiles_m = g.tiles_n = 0;
    bool strides4 = true;
    for (int k = 0; k < g.batch_rank; ++k) strides4 = strides4 && g.sa[k] % 4 == 0 && g.sb[k] % 4 == 0;
    g.vec = vec_operands(A, lda, B, ldb) && strides4;
    hipStream_t s = as_stream(stream);
    // 256x256 tiles once they alone fill every CU; 128x128 while those give at
    // least half as many workgroups as CUs; 64x64 (4 waves of 32x32) below.
    const size_t mid_tiles = ((M + 127) / 128) * ((N + 127) / 128) * batches;
    const unsigned nb = static_cast<unsigned>(batches);
    if (K >= 1 && K <= static_cast<size_t>(kBK) && g.batch_rank == 0 && !g.colsum) {  // one k tile
        launch_short_k(trans_a, trans_b, g, s);
    } else if (big_grid(M, N, batches)) {
        if (!g.vec) launch_tiles<256, 256, 2, 4>(trans_a, trans_b, g, s, nb);
        else launch_dma_layout(trans_a, trans_b, g, s, nb);
    } else if (2 * mid_tiles >= static_cast<size_t>(device_cu_count())) {
        launch_tiles<128, 128, 2, 2>(trans_a, trans_b, g, s, nb);
    } else {
        launch_tiles<64, 64, 2, 2>(trans_a, trans_b, g, s, nb);
    }
    return launch_status();
}

// ---- skinny products (N <= 16) -----------------------------------------------
//
// A product with at most 16 output columns over few rows and a long K (the
// narrow kernel below takes the rest) is a stream over A with N multiply-adds
// per element.  A workgroup of 4 waves takes 64 rows,
// a lane per row, and one slice of K (grid.y slices, enough row groups x
// slices for every CU); its waves split the slice into 4 contiguous ranges.
// A wave walks its range in chunks of 64 k: the chunk's B rows go to the
// wave's own LDS slab, zero-padded to 16 columns, its A values are loaded
// all at once, and each k then reads its B row as four broadcast float4s and
// does 16 fma on the lane's accumulators (k ascending).  The waves' sums are
// added in wave order through LDS; with one slice the result is stored with
// the epilogue, else slice s goes to P[s][M][N] and splitk_sum adds the slices
// in order and applies the epilogue.  Deterministic; the accumulation order
// differs from the MFMA kernels' (both within rounding of the exact product).
constexpr int kSkinnyN = 16;
constexpr int kSkinnyWaves = 4;
constexpr int kSkinnyChunk = 64;
constexpr int kSkinnyMaxSlices = 16;
static_assert(kSkinnyMaxSlices <= 16, "splitk_sum adds at most 16 slices");

template <bool TA, bool TB>
__global__ __launch_bounds__(64 * kSkinnyWaves) void gemm_skinny(GemmArgs g, float *P) {
    __shared__ float part[kSkinnyWaves][kSkinnyN][64];
    __shared__ float4 bs[kSkinnyWaves][kSkinnyChunk][kSkinnyN / 4];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int i = blockIdx.x * 64 + lane;
    const int ir = i < g.M ? i : g.M - 1;  // rows past M: an in-bounds row, never stored
    const float *__restrict__ A = g.A;
    const float *__restrict__ B = g.B;
    // k range of this wave within this workgroup's slice (slices are
    // g.kslice rows, a multiple of the column sum's chunk; wave ranges are
    // multiples of 4, so a row-major A row is read as float4)
    const int slices = gridDim.y, slice = blockIdx.y;
    const int ks = g.kslice;
    const int sb = min(g.K, slice * ks), se = min(g.K, sb + ks);
    const int kc = ((ks + kSkinnyWaves - 1) / kSkinnyWaves + 3) & ~3;
    const int kb = min(se, sb + wave * kc);
    const int ke = min(se, kb + kc);
    const int chunks = (kc + kSkinnyChunk - 1) / kSkinnyChunk;  // the same for every wave
    float acc[kSkinnyN];
#pragma unroll
    for (int j = 0; j < kSkinnyN; ++j) acc[j] = 0.0f;
    const float *arow = A + (size_t)ir * g.lda;
    const bool a4 = !TA && g.vec;
    for (int c = 0; c < chunks; ++c) {
        const int k0 = kb + c * kSkinnyChunk;
        const int len = max(0, min(kSkinnyChunk, ke - k0));  // uniform per wave
        // the chunk's A values first (they do not wait for the B slab), every
        // load of the chunk in flight at once, then the fma
        float av[kSkinnyChunk];
        if (len == kSkinnyChunk && a4) {  // row-major A: 4 k per dwordx4 load
#pragma unroll
            for (int q = 0; q < kSkinnyChunk / 4; ++q) {
                const float4 v = *reinterpret_cast<const float4 *>(arow + k0 + 4 * q);
                av[4 * q] = v.x;
                av[4 * q + 1] = v.y;
                av[4 * q + 2] = v.z;
                av[4 * q + 3] = v.w;
            }
        } else {  // A stored [K][lda]: the lanes read 64 consecutive floats per k
#pragma unroll
            for (int kk = 0; kk < kSkinnyChunk; ++kk)
                av[kk] = kk < len ? (TA ? A[(size_t)(k0 + kk) * g.lda + ir] : arow[k0 + kk]) : 0.0f;
        }
        // stage: lane l takes B row k0 + l, columns past N (and rows past the
        // range) as zeros
        {
            const int k = k0 + lane;
            float v[kSkinnyN];
#pragma unroll
            for (int j = 0; j < kSkinnyN; ++j)
                v[j] = (lane < len && j < g.N) ? (TB ? B[(size_t)j * g.ldb + k] : B[(size_t)k * g.ldb + j]) : 0.0f;
#pragma unroll
            for (int q = 0; q < kSkinnyN / 4; ++q)
                bs[wave][lane][q] = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kSkinnyChunk; ++kk) {
            if (kk < len) {  // uniform per wave
                const float4 b0 = bs[wave][kk][0], b1 = bs[wave][kk][1], b2 = bs[wave][kk][2], b3 = bs[wave][kk][3];
                const float b[kSkinnyN] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w,
                                           b2.x, b2.y, b2.z, b2.w, b3.x, b3.y, b3.z, b3.w};
#pragma unroll
                for (int j = 0; j < kSkinnyN; ++j) acc[j] = __builtin_fmaf(av[kk], b[j], acc[j]);
            }
        }
        __syncthreads();  // the slab is restaged next chunk
    }
#pragma unroll
    for (int j = 0; j < kSkinnyN; ++j) part[wave][j][lane] = acc[j];
    __syncthreads();
    if (i >= g.M) return;
    for (int j = wave; j < g.N; j += kSkinnyWaves) {
        float v = part[0][j][lane];
#pragma unroll
        for (int w = 1; w < kSkinnyWaves; ++w) v += part[w][j][lane];
        if (slices == 1) g.C[(size_t)i * g.ldc + j] = epilogue(g, v, i, j);
        else P[((size_t)slice * g.M + i) * g.N + j] = v;
    }
}

// ---- narrow products (N <= 16) in one pass ------------------------------------
//
// v_mfma_f32_16x16x4f32: lane l supplies A[l%16][l/16] of a 16x4 block and
// B[l/16][l%16] of a 4x16 block, and holds C[4*(l/16) + r][l%16] in its 4
// accumulators.  A workgroup owns a 16x16 block of C (grid.x over row blocks,
// grid.y over 16-column blocks: one column block for N <= 16) and all of K,
// split over its waves in contiguous ranges of whole 64-row chunks (the
// column sum's); B's columns past N are read clamped to column N-1 and feed
// outputs that are never stored.  A wave takes its range
// a chunk per round: four 16-k blocks, all their loads at once, then 16
// MFMAs.  Inside a block, lane group q = l/16 holds k = 4q .. 4q+3 and the
// block's MFMA s takes k = 4q + s (A and B follow the same order), so a
// row-major A row gives the lane its four k in one dwordx4.  The waves'
// accumulators are added in wave order through LDS and the epilogue applied
// at the store: one launch, no temporary.
// Column sums of B (CS, trans_b == 0): the first row block's workgroup of
// each column block holds every row of its 16 columns of B in its registers,
// a chunk per wave round, so each round also adds its chunk's rows in row
// order (lane j gathers column j's 64 values with cross-lane reads, f64 from
// +0), the chunk sums go to LDS, and 16 threads add them in the column sum's
// groups at the end.
// Used for N <= 16, and for products with few output tiles and a long K,
// while the blocks spread over the chip or K is moderate (with column sums in
// the kernel K <= kNarrowMaxK, the chunk table's size; past it a column-sum
// pass follows); past that the sliced skinny kernel above (N <= 16) or split-K
// takes them.
constexpr int kNarrowRows = 16;
constexpr int kNarrowMaxWaves = 16;
constexpr size_t kNarrowMaxK = 8192;
constexpr int kNarrowMaxChunks = static_cast<int>(kNarrowMaxK / kColsumRows);
static_assert(kColsumRows == 64, "a narrow wave round is one column-sum chunk");

// V: the k-contiguous operands (A unless TA, B when TB) take dwordx4 loads
// (16-byte aligned, leading dimension % 4 == 0).
// Workgroup (bx, by) of a gx-wide grid of narrow workgroups of
// blockDim.x threads (whole waves).
template <bool TA, bool TB, bool V, bool CS, bool XF>
__device__ __forceinline__ void narrow_block(const GemmArgs &g, int bx, int by, int gx) {
    static_assert(!CS || !TB, "column sums of B need trans_b == 0");
    if constexpr (CS) {
        // the row of workgroups appended for GemmArgs::sum_out (launched with
        // kNarrowMaxWaves waves): its first workgroup forms the sum
        if (g.sum_out && bx == gx - 1) {  // uniform
            if (by == 0) sum_in_workgroup<64 * kNarrowMaxWaves>(g);
            return;
        }
    }
    __shared__ float red[kNarrowMaxWaves][256];
    __shared__ double csum[CS ? kNarrowMaxChunks : 1][kSkinnyN];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int waves = blockDim.x >> 6;
    const int m0 = bx * kNarrowRows, n0 = by * kSkinnyN;
    const int q = lane >> 4;
    const int m = min(m0 + (lane & 15), g.M - 1);  // rows past M: never stored
    const int n = min(n0 + (lane & 15), g.N - 1);  // columns past N: never stored
    const int kc = ((g.K + waves - 1) / waves + 63) & ~63;
    const int kb = min(g.K, wave * kc), ke = min(g.K, kb + kc);
    const bool cs_wg = CS && bx == 0;  // uniform
    const XfRegs xfa = XF ? xf_load(g.xa) : XfRegs{}, xfb = XF ? xf_load(g.xb) : XfRegs{};
    const float *__restrict__ A = g.A;
    const float *__restrict__ B = g.B;
    auto a_at = [&](int k) { return TA ? A[(size_t)k * g.lda + m] : A[(size_t)m * g.lda + k]; };
    auto b_at = [&](int k) { return TB ? B[(size_t)n * g.ldb + k] : B[(size_t)k * g.ldb + n]; };
    // The epilogue's bias and mask values of the outputs this thread stores
    // (output t = 64r + l: row 4*(l/16) + r, column l%16), loaded now at
    // clamped addresses so they arrive with the operands.
    constexpr int kOuts = 256 / 64;
    float eb[kOuts] = {}, em[kOuts] = {}, es[kOuts] = {};
#pragma unroll
    for (int o = 0; o < kOuts; ++o) {
        if (o * static_cast<int>(blockDim.x) >= 256) break;  // uniform
        const int t = static_cast<int>(threadIdx.x) + o * static_cast<int>(blockDim.x);
        const int i = min(m0 + 4 * ((t & 63) >> 4) + ((t >> 6) & 3), g.M - 1), j = min(n0 + (t & 15), g.N - 1);
        eb[o] = g.bias ? g.bias[j] : 0.0f;
        em[o] = g.mask ? g.mask[(size_t)i * g.ldc + j] : 1.0f;
        es[o] = g.sub ? g.sub[(size_t)i * g.ldc + j] : 0.0f;
    }
    f4v_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = kb; k0 < ke; k0 += 64) {
        float av[4][4], bv[4][4];
        if (k0 + 64 <= ke) {  // a whole chunk (uniform)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int k = k0 + 16 * u + 4 * q;
                if (!TA && V) {
                    const f4v_t x = *reinterpret_cast<const f4v_t *>(A + (size_t)m * g.lda + k);
#pragma unroll
                    for (int s = 0; s < 4; ++s) av[u][s] = x[s];
                } else {
#pragma unroll
                    for (int s = 0; s < 4; ++s) av[u][s] = a_at(k + s);
                }
                if (TB && V) {
                    const f4v_t x = *reinterpret_cast<const f4v_t *>(B + (size_t)n * g.ldb + k);
#pragma unroll
                    for (int s = 0; s < 4; ++s) bv[u][s] = x[s];
                } else {
#pragma unroll
                    for (int s = 0; s < 4; ++s) bv[u][s] = b_at(k + s);
                }
            }
        } else {  // the last chunk of K: k past its end reads zeros
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const int k = k0 + 16 * u + 4 * q + s;
                    av[u][s] = k < ke ? a_at(k) : 0.0f;
                    bv[u][s] = k < ke ? b_at(k) : 0.0f;
                }
        }
        if constexpr (XF) {
            xf_each<16>(xfa, [&](int e) -> float & { return av[e / 4][e % 4]; });
            xf_each<16>(xfb, [&](int e) -> float & { return bv[e / 4][e % 4]; });
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u][s], bv[u][s], acc, 0, 0, 0);
        if (cs_wg) {
            // chunk k0/64: row r = 16u + 4q + s sits in lane (column, q) as
            // bv[u][s]; rows past K hold zeros, which add nothing to a sum
            // that starts at +0
            float v[64];
#pragma unroll
            for (int r = 0; r < 64; ++r) v[r] = __shfl(bv[r >> 4][r & 3], (lane & 15) + 16 * ((r >> 2) & 3));
            double sum = 0.0;
#pragma unroll
            for (int r = 0; r < 64; ++r) sum += (double)v[r];
            if (lane < kSkinnyN) csum[k0 >> 6][lane] = sum;
        }
    }
    // The mask values stay floats in registers until here: compared as soon
    // as they were loaded, each compare would wait for its load first.
#pragma unroll
    for (int o = 0; o < kOuts; ++o) asm volatile("" : "+v"(em[o]));
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][r * 64 + lane] = acc[r];
    __syncthreads();
#pragma unroll
    for (int o = 0; o < kOuts; ++o) {
        const int t = static_cast<int>(threadIdx.x) + o * static_cast<int>(blockDim.x);
        if (t >= 256) break;  // uniform per wave
        float v = red[0][t];
        for (int w = 1; w < waves; ++w) v += red[w][t];
        const int l = t & 63;
        const int i = m0 + 4 * (l >> 4) + (t >> 6), j = n0 + (l & 15);
        if (g.bias) v = v + eb[o];  // epilogue()'s order: bias, sub, relu, mask
        if (g.sub) v = v - es[o];
        if (g.relu) v = v > 0.0f ? v : 0.0f;
        if (g.mask) v = em[o] > 0.0f ? v : 0.0f;
        if (i < g.M && j < g.N) g.C[(size_t)i * g.ldc + j] = v;
    }
    if (cs_wg && static_cast<int>(threadIdx.x) < kSkinnyN && n0 + static_cast<int>(threadIdx.x) < g.N) {
        // the chunk sums in groups of kColsumGroup, each from +0
        constexpr int G = static_cast<int>(kColsumGroup);
        const int j = threadIdx.x, chunks = (g.K + 63) >> 6;
        double total = 0.0;
        for (int c0 = 0; c0 < chunks; c0 += G) {
            double x[G];
#pragma unroll
            for (int i = 0; i < G; ++i) x[i] = csum[min(c0 + i, chunks - 1)][j];
            double grp = 0.0;
#pragma unroll
            for (int i = 0; i < G; ++i)
                if (c0 + i < chunks) grp += x[i];
            total += grp;
        }
        g.colsum[n0 + j] = static_cast<float>(total);
    }
}

template <bool TA, bool TB, bool V, bool CS, bool XF = false>
__global__ __launch_bounds__(64 * kNarrowMaxWaves) void gemm_narrow(GemmArgs g) {
    narrow_block<TA, TB, V, CS, XF>(g, blockIdx.x, blockIdx.y, gridDim.x);
}

// A narrow product and a one-k-tile product in one launch (a launch group of
// the two; ts_hip_launch_group_begin): the first nb workgroups are the narrow
// product's (one row of column blocks, kNarrowMaxWaves waves), each later one
// runs tpw (1-4) of the other's 64x64 tiles, one per 256 threads.  The two
// write different outputs and read only inputs written before the launch.
template <bool NTA, bool NTB, bool NV, bool NCS, bool NXF, bool STA, bool STB, int SEPI, bool SXF>
__global__ __launch_bounds__(64 * kNarrowMaxWaves) void gemm_narrow_short_k(GemmArgs gn, GemmArgs gs, int nb,
                                                                             int tpw) {
    if (static_cast<int>(blockIdx.x) < nb) {  // uniform
        narrow_block<NTA, NTB, NV, NCS, NXF>(gn, blockIdx.x, 0, nb);
        return;
    }
    const int part = static_cast<int>(threadIdx.x >> 8);  // uniform per wave
    const int tile = (static_cast<int>(blockIdx.x) - nb) * tpw + part;
    if (part < tpw && tile < gs.tiles) short_k_tile<STA, STB, SEPI, SXF>(gs, tile, threadIdx.x & 255);
}

// Waves per narrow workgroup: the largest power of two up to 16 that leaves
// each wave at least 64 k.
static int narrow_waves(size_t K) {
    int w = 1;
    while (w < kNarrowMaxWaves && static_cast<size_t>(2 * w) * 64 <= K) w *= 2;
    return w;
}

static bool narrow_fits(size_t M, size_t N, size_t K) {
    const size_t blocks = ((M + kNarrowRows - 1) / kNarrowRows) * ((N + kSkinnyN - 1) / kSkinnyN);
    return K <= kNarrowMaxK || 8 * blocks >= static_cast<size_t>(device_cu_count());
}

template <bool TA, bool TB, bool V, bool CS, bool XF>
static void narrow_launch(dim3 grid, dim3 block, hipStream_t s, const GemmArgs &g) {
    hold_or_launch(kHeldNarrow, narrow_variant<TA, TB, V, CS, XF>(), gemm_narrow<TA, TB, V, CS, XF>, grid, block, s, g);
}

template <bool CS, bool XF>
static void launch_narrow_xf(int trans_a, int trans_b, bool v, const GemmArgs &g, dim3 grid, dim3 block,
                             hipStream_t s) {
    if (!trans_a && !trans_b) {
        if (v) narrow_launch<false, false, true, CS, XF>(grid, block, s, g);
        else narrow_launch<false, false, false, CS, XF>(grid, block, s, g);
    } else if (!trans_b) {
        narrow_launch<true, false, false, CS, XF>(grid, block, s, g);
    } else if (!CS) {  // column sums need trans_b == 0 (checked by the caller)
        if (!trans_a) {
            if (v) narrow_launch<false, true, true, false, XF>(grid, block, s, g);
            else narrow_launch<false, true, false, false, XF>(grid, block, s, g);
        } else {
            if (v) narrow_launch<true, true, true, false, XF>(grid, block, s, g);
            else narrow_launch<true, true, false, false, XF>(grid, block, s, g);
        }
    }
}

template <bool CS>
static void launch_narrow_as(int trans_a, int trans_b, bool v, const GemmArgs &g, dim3 grid, dim3 block,
                             hipStream_t s) {
    if (g.xa.n || g.xb.n) launch_narrow_xf<CS, true>(trans_a, trans_b, v, g, grid, block, s);
    else launch_narrow_xf<CS, false>(trans_a, trans_b, v, g, grid, block, s);
}

// g carries the epilogue and, optionally, colsum (trans_b == 0, K <= kNarrowMaxK).
static int launch_narrow(int trans_a, int trans_b, size_t M, size_t N, size_t K, const float *A, size_t lda,
                         const float *B, size_t ldb, float *C, size_t ldc, GemmArgs g, void *stream) {
    if (!A || !B) return TS_HIP_EINVAL;
    if (lda < (trans_a ? M : K) || ldb < (trans_b ? K : N)) return TS_HIP_EINVAL;
    const size_t lim = 0x7ffffe00ULL;
    if (M > lim || N > lim || K > lim || lda > lim || ldb > lim || ldc > lim) return TS_HIP_EINVAL;
    if ((N + kSkinnyN - 1) / kSkinnyN > 65535) return TS_HIP_EINVAL;  // grid.y
    if (g.colsum && (trans_b || K > kNarrowMaxK)) return TS_HIP_EINVAL;
    g.A = A; g.B = B; g.C = C;
    g.M = static_cast<int>(M); g.N = static_cast<int>(N); g.K = static_cast<int>(K);
    g.lda = static_cast<int>(lda); g.ldb = static_cast<int>(ldb); g.ldc = static_cast<int>(ldc);
    const bool va = trans_a || (aligned16(A) && lda % 4 == 0);
    const bool vb = !trans_b || (aligned16(B) && ldb % 4 == 0);
    // the sum's workgroup: a row block appended (full width, kNarrowMaxWaves waves)
    if (g.sum_out && (!g.colsum || narrow_waves(K) != kNarrowMaxWaves)) return TS_HIP_EINVAL;
    const dim3 grid(static_cast<unsigned>((M + kNarrowRows - 1) / kNarrowRows + (g.sum_out ? 1 : 0)),
                    static_cast<unsigned>((N + kSkinnyN - 1) / kSkinnyN)),
        block(64 * narrow_waves(K));
    hipStream_t s = as_stream(stream);
    if (g.colsum) launch_narrow_as<true>(trans_a, trans_b, va && vb, g, grid, block, s);
    else launch_narrow_as<false>(trans_a, trans_b, va && vb, g, grid, block, s);
    return launch_status();
}

using PairKernel = void (*)(GemmArgs, GemmArgs, int, int);

// The instantiated pairs: an MLP backward's dW of a layer with few outputs
// (narrow, A transposed, with the bias gradient's column sums) and its dX
// (one k tile, B transposed, relu-backward mask), with and without operand
// transforms on the gradient they share.
static PairKernel pair_kernel(int nv, int sv) {
    if (nv == narrow_variant<true, false, false, true, true>() && sv == short_k_variant<false, true, kEpiAll, true>())
        return gemm_narrow_short_k<true, false, false, true, true, false, true, kEpiAll, true>;
    if (nv == narrow_variant<true, false, false, true, false>() && sv == short_k_variant<false, true, kEpiAll, false>())
        return gemm_narrow_short_k<true, false, false, true, false, false, true, kEpiAll, false>;
    return nullptr;
}

extern "C" int ts_hip_launch_group_begin(void *stream) {
    tship::LaunchGroupState &lg = tship::t_group;
    if (lg.open) return TS_HIP_EINVAL;
    lg.open = true;
    lg.stream = tship::as_stream(stream);
    lg.n = 0;
    return TS_HIP_OK;
}

extern "C" int ts_hip_launch_group_end(void *stream) {
    using namespace tship;
    LaunchGroupState &lg = t_group;
    if (!lg.open || lg.stream != as_stream(stream)) return TS_HIP_EINVAL;
    lg.open = false;
    if (lg.n == 2 && lg.held[0].kind != lg.held[1].kind) {
        const HeldLaunch &nr = lg.held[0].kind == kHeldNarrow ? lg.held[0] : lg.held[1];
        const HeldLaunch &sk = lg.held[0].kind == kHeldNarrow ? lg.held[1] : lg.held[0];
        const PairKernel k = pair_kernel(nr.variant, sk.variant);
        if (k && nr.grid.y == 1 && nr.block.x == 64 * kNarrowMaxWaves) {
            lg.n = 0;
            // one workgroup of either kind per CU (the narrow one holds a CU
            // at its register count): the one-k-tile product's tiles over the
            // CUs the narrow product leaves, up to four per workgroup
            const int nb = static_cast<int>(nr.grid.x), free = device_cu_count() - nb;
            int tpw = 1;
            while (tpw < 4 && (free <= 0 || static_cast<long long>(free) * tpw < sk.g.tiles)) tpw *= 2;
            const unsigned sb = static_cast<unsigned>((sk.g.tiles + tpw - 1) / tpw);
            launch_now(k, dim3(static_cast<unsigned>(nb) + sb), dim3(64 * kNarrowMaxWaves), 0, lg.stream, nr.g, sk.g,
                       nb, tpw);
            return launch_status();
        }
    }
    flush_launch_group();
    return launch_status();
}

static bool skinny(size_t N) { return N <= static_cast<size_t>(kSkinnyN); }

// Slices of K for a skinny product: enough (row group x slice) workgroups for
// every CU, each slice at least 64 k long; 1 when the row groups alone
// fill the chip.
// Rows per slice for a wanted slice count, a whole number of the column sum's
// chunks.
static size_t skinny_kslice(size_t K, size_t sl) {
    const size_t per = (K + sl - 1) / sl;
    return (per + kColsumRows - 1) / kColsumRows * kColsumRows;
}

static int skinny_slices(size_t M, size_t K) {
    const size_t cus = static_cast<size_t>(device_cu_count());
    const size_t groups = (M + 63) / 64;
    if (groups >= cus || K == 0) return 1;
    size_t sl = (cus + groups - 1) / groups;
    if (sl > static_cast<size_t>(kSkinnyMaxSlices)) sl = kSkinnyMaxSlices;
    const size_t by_k = K / 64 > 0 ? K / 64 : 1;
    if (sl > by_k) sl = by_k;
    const size_t ks = skinny_kslice(K, sl);
    return static_cast<int>((K + ks - 1) / ks);  // slices that hold rows
}

// P: slices * M * N floats when skinny_slices(M, K) > 1 (else unused).
// With g.colsum set and one slice, g.colsum_part holds colsum_chunk_count(K) * N
// doubles for the column-sum pass.
static int launch_skinny(int trans_a, int trans_b, size_t M, size_t N, size_t K, const float *A, size_t lda,
                         const float *B, size_t ldb, float *C, size_t ldc, GemmArgs g, float *P, void *stream) {
    if (!A || !B) return TS_HIP_EINVAL;
    if (lda < (trans_a ? M : K) || ldb < (trans_b ? K : N)) return TS_HIP_EINVAL;
    const size_t lim = 0x7ffffe00ULL;
    if (M > lim || K > lim || lda > lim || ldb > lim || ldc > lim) return TS_HIP_EINVAL;
    const int slices = skinny_slices(M, K);
    if (slices > 1 && !P) return TS_HIP_EINVAL;
    if (g.colsum && !g.colsum_part) return TS_HIP_EINVAL;
    g.A = A; g.B = B; g.C = C;
    g.M = static_cast<int>(M); g.N = static_cast<int>(N); g.K = static_cast<int>(K);
    g.lda = static_cast<int>(lda); g.ldb = static_cast<int>(ldb); g.ldc = static_cast<int>(ldc);
    g.vec = aligned16(A) && (lda % 4 == 0);
    g.kslice = static_cast<int>(skinny_kslice(K, static_cast<size_t>(slices)));
    if (!g.colsum) g.colsum_part = nullptr;
    const dim3 grid(static_cast<unsigned>((M + 63) / 64), static_cast<unsigned>(slices)), block(64 * kSkinnyWaves);
    hipStream_t s = as_stream(stream);
    if (g.colsum && trans_b) return TS_HIP_EINVAL;
    if (!trans_a && !trans_b) launch((gemm_skinny<false, false>), grid, block, 0, s, g, P);
    else if (!trans_a) launch((gemm_skinny<false, true>), grid, block, 0, s, g, P);
    else if (!trans_b) launch((gemm_skinny<true, false>), grid, block, 0, s, g, P);
    else launch((gemm_skinny<true, true>), grid, block, 0, s, g, P);
    int st = launch_status();
    if (st != TS_HIP_OK) return st;
    if (slices == 1)  // the column sums as a pass of their own
        return g.colsum ? launch_colsum(B, nullptr, K, N, ldb, g.colsum, reinterpret_cast<float *>(g.colsum_part),
                                        2 * colsum_chunk_count(K) * N, stream)
                        : TS_HIP_OK;
    // the slice sum; with column sums, one more workgroup adds B's columns
    const size_t blocks = (M * N + kBlock - 1) / kBlock + (g.colsum ? 1 : 0);
    launch(splitk_sum, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, P, slices, M, N, C, ldc, g);
    return launch_status();
}

// Few output tiles and a long K: K is split into this many slices (1: not
// split), computed as a batch into a temporary of slices*M*N floats and then
// added in slice order.
static int split_slices(size_t M, size_t N, size_t K) {
    if (skinny(N)) return skinny_slices(M, K);
    const size_t cus = static_cast<size_t>(device_cu_count());
    const size_t tiles64 = ((M + 63) / 64) * ((N + 63) / 64);
    if (4 * tiles64 < cus && K >= 512) {
        for (int sl : {16, 8, 4, 2}) {
            if (K % sl == 0 && K / sl >= 32 && tiles64 * sl <= 2 * cus) return sl;
        }
    }
    return 1;
}

// Workspace of one product: the split temporary (slices * M * N floats) and,
// with column sums of B, colsum_chunk_count(K) * N doubles of chunk sums after
// it (8-byte aligned) -- written by the LDS-DMA kernel (then added by
// colsum_final) or by a column-sum pass after the product.  The narrow kernel
// and the register-staged tiles (column strips in their own grid) write the
// column sums directly.
struct GemmPlan {
    bool skinny = false;
    bool narrow = false;  // the narrow kernel: one pass, no temporary (N <= 16, or few tiles and a long K)
    int slices = 1;
    size_t split_floats = 0;
    size_t part_floats = 0;
    bool cs_kernel = false;  // the product's kernels write the column sums
    size_t part_offset() const { return (split_floats + 1) & ~size_t(1); }
    size_t total() const { return part_floats ? part_offset() + part_floats : split_floats; }
};

static GemmPlan gemm_plan(int trans_a, int trans_b, size_t M, size_t N, size_t K, bool colsum) {
    GemmPlan p;
    if (M == 0 || N == 0 || K == 0) return p;
    p.skinny = skinny(N);
    // the narrow kernel for N <= 16, and for the few-tile, long-K shapes split-K
    // takes otherwise (the same kernel with or without column sums)
    const size_t tiles64 = ((M + 63) / 64) * ((N + 63) / 64);
    const bool few_tiles = !p.skinny && 4 * tiles64 < static_cast<size_t>(device_cu_count()) && K >= 512;
    p.narrow = (p.skinny || few_tiles) && narrow_fits(M, N, K);
    p.slices = p.narrow ? 1 : p.skinny ? skinny_slices(M, K) : split_slices(M, N, K);
    p.split_floats = p.slices > 1 ? static_cast<size_t>(p.slices) * M * N : 0;
    p.cs_kernel = colsum && (p.narrow ? K <= kNarrowMaxK : !p.skinny && p.slices == 1 && trans_a && !trans_b);
    // chunk sums in the workspace: a column-sum pass's, or the LDS-DMA kernel's
    // (sized whenever the grid could take that kernel: alignment is not known here)
    const bool dma_cs = p.cs_kernel && !p.narrow && big_grid(M, N, 1);
    p.part_floats = colsum && (!p.cs_kernel || dma_cs) ? 2 * colsum_chunk_count(K) * N : 0;
    return p;
}

// Whether the kernels a product takes apply operand transforms: one pass of
// the narrow, one-k-tile or register-staged kernels (fewer 256x256 tiles
// than CUs, so never the LDS-DMA kernel), with its column sums (if any)
// written by that pass.
static bool xf_plan_ok(const GemmPlan &p, size_t M, size_t N, size_t K, bool colsum) {
    if (M == 0 || N == 0 || K == 0) return true;
    return !big_grid(M, N, 1) && p.slices == 1 && (p.narrow || !p.skinny) && (!colsum || p.cs_kernel);
}

// A caller's transform checked (codes, op count, +0 -> +0) and copied.
static bool xf_from(const ts_hip_operand_xf *x, OperandXf &out) {
    out = OperandXf{};
    if (!x || x->n_ops == 0) return true;
    if (x->n_ops > TS_HIP_XF_MAX_OPS) return false;
    float v = 0.0f;
    for (uint32_t i = 0; i < x->n_ops; ++i) {
        const float c = x->imm[i];
        switch (x->code[i]) {
            case TS_HIP_XF_ADD_S: v = v + c; break;
            case TS_HIP_XF_SUB_S: v = v - c; break;
            case TS_HIP_XF_MUL_S: v = v * c; break;
            case TS_HIP_XF_DIV_S: v = v / c; break;
            case TS_HIP_XF_RSUB_S: v = c - v; break;
            case TS_HIP_XF_RDIV_S: v = c / v; break;
            case TS_HIP_XF_RELU: v = v > 0.0f ? v : 0.0f; break;
            case TS_HIP_XF_RELU_BWD_S: v = v > 0.0f ? c : 0.0f; break;
            case TS_HIP_XF_SQUARE: v = v * v; break;
            default: return false;
        }
        out.code[i] = x->code[i];
        out.imm[i] = c;
    }
    uint32_t bits;
    std::memcpy(&bits, &v, 4);
    if (bits != 0) return false;  // +0 must stay +0
    out.n = static_cast<int>(x->n_ops);
    return true;
}

// One 2-D product with an optional epilogue (GemmArgs::bias / mask / relu)
// and optional column sums of B (colsum, trans_b == 0, no epilogue), its
// operands optionally transformed as loaded (xa, xb: null or n == 0 for
// none).  The workspace is `ws` when given (at least gemm_plan(...).total()
// floats), else it comes from the stream-ordered allocator.
static int gemm_plain(int trans_a, int trans_b, size_t M, size_t N, size_t K, const float *A, size_t lda,
                      const float *B, size_t ldb, float *C, size_t ldc, const float *bias, const float *mask,
                      int relu, float *colsum, float *ws, size_t ws_floats, void *stream,
                      const OperandXf *xa = nullptr, const OperandXf *xb = nullptr) {
    if (M == 0 || N == 0) return TS_HIP_OK;
    if (!C || ldc < N) return TS_HIP_EINVAL;
    if (colsum && (trans_b || bias || mask || relu)) return TS_HIP_EINVAL;
    const bool xf = (xa && xa->n) || (xb && xb->n);
    if (xf && !xf_plan_ok(gemm_plan(trans_a, trans_b, M, N, K, colsum != nullptr), M, N, K, colsum != nullptr))
        return TS_HIP_EINVAL;
    if (K == 0) {  // empty contraction: C = 0, then the epilogue
        if (ldc != N) return TS_HIP_EINVAL;
        int st = ts_hip_fill(C, 0.0f, M * N, stream);
        if (st == TS_HIP_OK && bias) st = ts_hip_row_broadcast(0, C, bias, C, M, N, 0, 0, nullptr, stream);
        if (st == TS_HIP_OK && relu) st = ts_hip_relu(C, C, M * N, stream);
        if (st == TS_HIP_OK && mask) st = ts_hip_relu_backward(mask, C, C, M * N, stream);
        if (st == TS_HIP_OK && colsum) st = ts_hip_fill(colsum, 0.0f, N, stream);
        return st;
    }
    if (!A || !B || lda < (trans_a ? M : K) || ldb < (trans_b ? K : N)) return TS_HIP_EINVAL;
    const GemmPlan plan = gemm_plan(trans_a, trans_b, M, N, K, colsum != nullptr);
    const size_t need = plan.total();
    hipStream_t st = as_stream(stream);
    float *W = ws;
    bool owned = false;
    if (need && ws && (ws_floats < need || (plan.part_floats && (reinterpret_cast<uintptr_t>(ws) & 7u))))
        return TS_HIP_EWORKSPACE;
    if (need && !W) {
        const hipError_t ae = hipMallocAsync(reinterpret_cast<void **>(&W), need * sizeof(float), st);
        if (ae == hipSuccess) {
            owned = true;
        } else {
            (void)hipGetLastError();
            W = nullptr;
            // no stream-ordered memory: an MFMA split runs unsplit; the rest
            // needs memory, and the allocator's error is returned
            // (hipErrorOutOfMemory when the device is full)
            if ((plan.skinny && plan.slices > 1) || plan.part_floats) return static_cast<int>(ae);
        }
    }
    double *part = plan.part_floats ? reinterpret_cast<double *>(W + plan.part_offset()) : nullptr;
    int status;
    if (plan.narrow) {  // few output columns, or few output tiles and a long K: one pass
        GemmArgs g{};
        g.bias = bias;
        g.mask = mask;
        g.relu = relu;
        if (xa) g.xa = *xa;
        if (xb) g.xb = *xb;
        if (plan.cs_kernel) g.colsum = colsum;
        status = launch_narrow(trans_a, trans_b, M, N, K, A, lda, B, ldb, C, ldc, g, stream);
        if (status == TS_HIP_OK && colsum && !plan.cs_kernel)  // K past the kernel's chunk table
            status = launch_colsum(B, nullptr, K, N, ldb, colsum, reinterpret_cast<float *>(part), plan.part_floats,
                                   stream);
    } else if (plan.skinny) {  // few output columns over few rows: K split over the CUs
        GemmArgs g{};
        g.bias = bias;
        g.mask = mask;
        g.relu = relu;
        g.colsum = colsum;
        g.colsum_part = part;
        status = launch_skinny(trans_a, trans_b, M, N, K, A, lda, B, ldb, C, ldc, g, W, stream);
    } else if (plan.slices > 1 && W) {
        const int slices = plan.slices;
        const size_t kc = K / slices;
        GemmArgs e{};  // epilogue after the slice sum
        e.bias = bias;
        e.mask = mask;
        e.relu = relu;
        e.ldc = static_cast<int>(ldc);
        GemmArgs g{};
        g.batch_rank = 1;
        g.bdims[0] = slices;
        g.sa[0] = static_cast<long long>(trans_a ? kc * lda : kc);
        g.sb[0] = static_cast<long long>(trans_b ? kc : kc * ldb);
        g.sc = static_cast<long long>(M * N);
        status = gemm_launch(trans_a, trans_b, M, N, kc, A, lda, B, ldb, W, N, g, slices, stream);
        if (status == TS_HIP_OK) {
            const size_t blocks = (M * N + kBlock - 1) / kBlock;
            launch(splitk_sum, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, st, W, slices, M, N, C, ldc, e);
            status = launch_status();
        }
        if (status == TS_HIP_OK && colsum)
            status = launch_colsum(B, nullptr, K, N, ldb, colsum, reinterpret_cast<float *>(part), plan.part_floats,
                                   stream);
    } else {
        GemmArgs g{};
        g.bias = bias;
        g.mask = mask;
        g.relu = relu;
        if (xa) g.xa = *xa;
        if (xb) g.xb = *xb;
        if (plan.cs_kernel) {
            g.colsum = colsum;
            g.colsum_part = part;
        }
        status = gemm_launch(trans_a, trans_b, M, N, K, A, lda, B, ldb, C, ldc, g, 1, stream);
        if (status == TS_HIP_OK && plan.cs_kernel && big_grid(M, N, 1) && vec_operands(A, lda, B, ldb))
            status = launch_colsum_final(part, colsum_chunk_count(K), N, colsum, st);  // the DMA kernel's chunks
        else if (status == TS_HIP_OK && colsum && !plan.cs_kernel)  // (register tiles: written by their strips)
            status = launch_colsum(B, nullptr, K, N, ldb, colsum, reinterpret_cast<float *>(part), plan.part_floats,
                                   stream);
    }
    if (!owned) return status;
    const hipError_t fe = hipFreeAsync(W, st);
    return status != TS_HIP_OK ? status : static_cast<int>(fe);
}

extern "C" int ts_hip_gemm(int trans_a, int trans_b, size_t M, size_t N, size_t K, const float *A,
                           size_t lda, const float *B, size_t ldb, float *C, size_t ldc,
                           void *stream) {
    return gemm_plain(trans_a, trans_b, M, N, K, A, lda, B, ldb, C, ldc, nullptr, nullptr, 0, nullptr, nullptr, 0,
                      stream);
}

// ---- allocation-free form --------------------------------------------------
//
// ts_hip_gemm_noalloc takes the split-K temporary from this fixed device
// array instead of the stream-ordered allocator.  An MFMA split runs only
// while 4 * (64x64 tiles) < CUs with slices * tiles <= 2 * CUs, so it never
// needs more than 2 * CUs * 64 * 64 floats: 2^21 (8 MiB) on the 256 CUs of an
// MI355X; a skinny split (N <= 16) has fewer 64-row groups than CUs and at
// most CUs / groups + 1 slices, so slices * M * N <= 128 * CUs * 16 = 2^19.  Every device the library runs on holds its own copy for the life
// of the process.  Calls that overlap on one device (several streams) share
// it and race; the split slices are fully written before they are read, so
// nothing needs clearing between calls.
static constexpr size_t kScratchFloats = size_t(1) << 21;
static __device__ __align__(256) float scratch[kScratchFloats];

namespace tship {
static std::mutex g_scratch_mutex;
static std::vector<float *> g_scratch;  // device ordinal -> this device's copy of `scratch`

// The device address of the current device's copy of `scratch`, looked up
// once per device with that device current (host code must never pass the
// symbol itself: on the host it names a host-side stand-in).
static int scratch_address(float **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return static_cast<int>(e);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (static_cast<size_t>(dev) >= g_scratch.size()) g_scratch.resize(dev + 1, nullptr);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return e != hipSuccess ? static_cast<int>(e) : TS_HIP_EINVAL;
        g_scratch[dev] = static_cast<float *>(p);
    }
    *out = g_scratch[dev];
    return TS_HIP_OK;
}
}  // namespace tship

extern "C" int ts_hip_gemm_noalloc(int trans_a, int trans_b, size_t M, size_t N, size_t K, const float *A,
                                   size_t lda, const float *B, size_t ldb, float *C, size_t ldc, void *stream) {
    const size_t need = ts_hip_gemm_workspace_floats(M, N, K);
    if (need > kScratchFloats) return TS_HIP_ESCRATCH;
    float *ws = nullptr;
    if (need) {
        const int st = scratch_address(&ws);
        if (st != TS_HIP_OK) return st;
    }
    // with a workspace given, a split product takes its temporary from it;
    // unsplit products and empty contractions use none
    return gemm_plain(trans_a, trans_b, M, N, K, A, lda, B, ldb, C, ldc, nullptr, nullptr, 0, nullptr, ws, need,
                      stream);
}

extern "C" size_t ts_hip_gemm_workspace_floats(size_t M, size_t N, size_t K) {
    return gemm_plan(0, 0, M, N, K, false).total();
}

extern "C" int ts_hip_gemm_fused(int trans_a, int trans_b, size_t M, size_t N, size_t K, const float *A,
                                 size_t lda, const float *B, size_t ldb, const float *bias, int relu,
                                 const float *mask, float *C, size_t ldc, float *workspace,
                                 size_t workspace_floats, void *stream) {
    return gemm_plain(trans_a, trans_b, M, N, K, A, lda, B, ldb, C, ldc, bias, mask, relu != 0, nullptr, workspace,
                      workspace_floats, stream);
}

extern "C" size_t ts_hip_gemm_colsum_workspace_floats(int trans_a, size_t M, size_t N, size_t K) {
    if (N == 0 || K == 0) return 0;
    if (M == 0) return 2 * colsum_chunk_count(K) * N;  // the column sums alone
    return gemm_plan(trans_a, 0, M, N, K, true).total();
}

extern "C" int ts_hip_gemm_colsum(int trans_a, size_t M, size_t N, size_t K, const float *A, size_t lda,
                                  const float *B, size_t ldb, float *C, size_t ldc, float *colsum, float *workspace,
                                  size_t workspace_floats, void *stream) {
    if (!colsum) return TS_HIP_EINVAL;
    if (N == 0) return TS_HIP_OK;
    if (M == 0) {  // no product, the column sums alone
        if (K == 0) return ts_hip_fill(colsum, 0.0f, N, stream);
        if (!B || ldb < N) return TS_HIP_EINVAL;
        const size_t need = 2 * colsum_chunk_count(K) * N;
        if (workspace) {
            if (workspace_floats < need) return TS_HIP_EWORKSPACE;
            return launch_colsum(B, nullptr, K, N, ldb, colsum, workspace, workspace_floats, stream);
        }
        hipStream_t st = as_stream(stream);
        float *W = nullptr;
        const hipError_t ae = hipMallocAsync(reinterpret_cast<void **>(&W), need * sizeof(float), st);
        if (ae != hipSuccess) {
            (void)hipGetLastError();
            return static_cast<int>(ae);  // hipErrorOutOfMemory when the device is full
        }
        const int status = launch_colsum(B, nullptr, K, N, ldb, colsum, W, need, stream);
        const hipError_t fe = hipFreeAsync(W, st);
        return status != TS_HIP_OK ? status : static_cast<int>(fe);
    }
    return gemm_plain(trans_a, 0, M, N, K, A, lda, B, ldb, C, ldc, nullptr, nullptr, 0, colsum, workspace,
                      workspace_floats, stream);
}

extern "C" int ts_hip_gemm_takes_sub(int trans_a, int trans_b, size_t M, size_t N, size_t K) {
    if (M == 0 || N == 0 || K == 0) return 0;
    return gemm_plan(trans_a, trans_b, M, N, K, false).narrow ? 1 : 0;
}

extern "C" int ts_hip_gemm_fused_sub(int trans_a, int trans_b, size_t M, size_t N, size_t K, const float *A,
                                     size_t lda, const float *B, size_t ldb, const float *bias, const float *sub,
                                     int relu, const float *mask, float *C, size_t ldc, void *stream) {
    if (!ts_hip_gemm_takes_sub(trans_a, trans_b, M, N, K) || !sub || !C || ldc < N) return TS_HIP_EINVAL;
    GemmArgs g{};
    g.bias = bias;
    g.sub = sub;
    g.relu = relu != 0;
    g.mask = mask;
    return launch_narrow(trans_a, trans_b, M, N, K, A, lda, B, ldb, C, ldc, g, stream);
}

extern "C" int ts_hip_gemm_takes_bsum(int trans_a, size_t M, size_t N, size_t K) {
    if (!trans_a || M == 0 || N == 0 || K == 0) return 0;
    const GemmPlan p = gemm_plan(1, 0, M, N, K, true);
    // the register-staged tiles with their column strips (one pass, no
    // temporary), or the narrow kernel with its column sums and its widest
    // workgroups; and a B that one workgroup's sum covers
    const bool strips = !p.narrow && !p.skinny && p.slices == 1 && p.cs_kernel && !big_grid(M, N, 1) && p.total() == 0;
    const bool narrow = p.narrow && p.cs_kernel && narrow_waves(K) == kNarrowMaxWaves;
    const size_t n = K * N;
    return (strips || narrow) && n / K == N && sum_blocks(n) <= static_cast<size_t>(kSumSmallBlocks) ? 1 : 0;
}

extern "C" int ts_hip_gemm_colsum_bsum(int trans_a, size_t M, size_t N, size_t K, const float *A, size_t lda,
                                       const ts_hip_operand_xf *xa, const float *B, const ts_hip_operand_xf *xb,
                                       float *C, size_t ldc, float *colsum, const ts_hip_operand_xf *xs,
                                       float *bsum, int mean, void *stream) {
    if (!ts_hip_gemm_takes_bsum(trans_a, M, N, K) || !A || !B || !C || !colsum || !bsum || ldc < N)
        return TS_HIP_EINVAL;
    if (!aligned16(B) && K * N >= 4) return TS_HIP_EINVAL;  // the sum's float4 loads
    OperandXf fa, fb;
    GemmArgs g{};
    if (!xf_from(xa, fa) || !xf_from(xb, fb) || !xf_from(xs, g.sum_xf)) return TS_HIP_EINVAL;
    g.xa = fa;
    g.xb = fb;
    g.colsum = colsum;
    g.sum_x = B;  // as stored: xb applies to the product's loads, xs to the summed values
    g.sum_out = bsum;
    g.sum_n = K * N;
    g.sum_mean = mean != 0;
    g.sum_blocks = static_cast<int>(sum_blocks(K * N));
    if (gemm_plan(1, 0, M, N, K, true).narrow) return launch_narrow(1, 0, M, N, K, A, lda, B, N, C, ldc, g, stream);
    return gemm_launch(1, 0, M, N, K, A, lda, B, N, C, ldc, g, 1, stream);
}

extern "C" int ts_hip_gemm_takes_xf(int trans_a, int trans_b, size_t M, size_t N, size_t K, int colsum) {
    return xf_plan_ok(gemm_plan(trans_a, trans_b, M, N, K, colsum != 0), M, N, K, colsum != 0) ? 1 : 0;
}

extern "C" int ts_hip_gemm_fused_xf(int trans_a, int trans_b, size_t M, size_t N, size_t K, const float *A,
                                    size_t lda, const ts_hip_operand_xf *xa, const float *B, size_t ldb,
                                    const ts_hip_operand_xf *xb, const float *bias, int relu, const float *mask,
                                    float *C, size_t ldc, float *workspace, size_t workspace_floats,
                                    void *stream) {
    OperandXf fa, fb;
    if (!xf_from(xa, fa) || !xf_from(xb, fb)) return TS_HIP_EINVAL;
    return gemm_plain(trans_a, trans_b, M, N, K, A, lda, B, ldb, C, ldc, bias, mask, relu != 0, nullptr, workspace,
                      workspace_floats, stream, &fa, &fb);
}

extern "C" int ts_hip_gemm_colsum_xf(int trans_a, size_t M, size_t N, size_t K, const float *A, size_t lda,
                                     const ts_hip_operand_xf *xa, const float *B, size_t ldb,
                                     const ts_hip_operand_xf *xb, float *C, size_t ldc, float *colsum,
                                     float *workspace, size_t workspace_floats, void *stream) {
    OperandXf fa, fb;
    if (!xf_from(xa, fa) || !xf_from(xb, fb)) return TS_HIP_EINVAL;
    if (!fa.n && !fb.n)  // no transform: the plain call
        return ts_hip_gemm_colsum(trans_a, M, N, K, A, lda, B, ldb, C, ldc, colsum, workspace, workspace_floats,
                                  stream);
    if (!colsum || M == 0) return TS_HIP_EINVAL;  // the column sums alone take no transform
    if (N == 0) return TS_HIP_OK;
    return gemm_plain(trans_a, 0, M, N, K, A, lda, B, ldb, C, ldc, nullptr, nullptr, 0, colsum, workspace,
                      workspace_floats, stream, &fa, &fb);
}

extern "C" int ts_hip_gemm_batched(int trans_a, int trans_b, size_t M, size_t N, size_t K, const float *A,
                                   size_t lda, const float *B, size_t ldb, float *C, size_t ldc,
                                   size_t batch_rank, const size_t *batch_dims, const size_t *a_batch_strides,
                                   const size_t *b_batch_strides, size_t c_batch_stride, void *stream) {
    if (batch_rank > static_cast<size_t>(kMaxBatchRank)) return TS_HIP_EINVAL;
    if (batch_rank && (!batch_dims || !a_batch_strides || !b_batch_strides)) return TS_HIP_EINVAL;
    size_t batches = 1;
    for (size_t k = 0; k < batch_rank; ++k) batches *= batch_dims[k];
    if (M == 0 || N == 0 || batches == 0) return TS_HIP_OK;
    if (!C || ldc < N || c_batch_stride < (M - 1) * ldc + N) return TS_HIP_EINVAL;
    if (K == 0) {  // empty contraction: every C batch = 0
        if (ldc != N || c_batch_stride != M * N) return TS_HIP_EINVAL;
        return ts_hip_fill(C, 0.0f, batches * M * N, stream);
    }
    if (batches > 0x7fffffffULL) return TS_HIP_EINVAL;
    GemmArgs g{};
    g.batch_rank = static_cast<int>(batch_rank);
    for (size_t k = 0; k < batch_rank; ++k) {
        if (batch_dims[k] > 0x7fffffffULL) return TS_HIP_EINVAL;
        g.bdims[k] = static_cast<int>(batch_dims[k]);
        g.sa[k] = static_cast<long long>(a_batch_strides[k]);
        g.sb[k] = static_cast<long long>(b_batch_strides[k]);
    }
    g.sc = static_cast<long long>(c_batch_stride);
    return gemm_launch(trans_a, trans_b, M, N, K, A, lda, B, ldb, C, ldc, g, batches, stream);
}

extern "C" int ts_hip_matmul(const float *a, const float *b, float *c, size_t m, size_t n, size_t k,
                             void *stream) {
    return ts_hip_gemm(0, 0, m, n, k, a, k, b, n, c, n, stream);
}
