// Device-side random initialisation: Tensor::randn / fill_randn
// (tensor/init/random.rs:231-299) with the reference's XorShiftRng
// (random.rs:453-615), generated on the GPU instead of uploaded.
//
// Element i of randn(seed) is Box-Muller on draws 2i+1 and 2i+2 of
// xorshift64(13, 7, 17) started at `seed`.  The generator is linear over
// GF(2)^64, s_k = M^k s_0, so every thread can start at its own draw index:
// kJump holds the 64 columns of M^(2^j) for j = 0..63 (built at compile time
// by repeated squaring), and reaching draw d costs one GF(2) matrix-vector
// product per set bit of d.  A thread then generates a contiguous run of
// elements sequentially, exactly as the reference's single generator would.
//
// ln and cos are evaluated in f64 and rounded once to f32, which is correctly
// rounded on every input the generator can produce (u in [0.5, 1), 2^23
// values per function).  The reference calls the host libm's logf / cosf;
// where those are not correctly rounded the two differ in the last place of
// that intermediate.
#include "ts_hip_internal.h"
#include "ts_hip_libm.h"

namespace tship {

struct JumpTable {
    uint64_t col[64][64];  // col[j][b] = M^(2^j) e_b
};

constexpr uint64_t xs_step(uint64_t s) {
    s ^= s << 13;
    s ^= s >> 7;
    s ^= s << 17;
    return s;
}

constexpr uint64_t gf2_apply(const uint64_t (&col)[64], uint64_t s) {
    uint64_t r = 0;
    for (int b = 0; b < 64; ++b)
        if ((s >> b) & 1u) r ^= col[b];
    return r;
}

constexpr JumpTable make_jump_table() {
    JumpTable t{};
    for (int b = 0; b < 64; ++b) t.col[0][b] = xs_step(uint64_t(1) << b);
    for (int j = 1; j < 64; ++j)
        for (int b = 0; b < 64; ++b) t.col[j][b] = gf2_apply(t.col[j - 1], t.col[j - 1][b]);
    return t;
}

__constant__ JumpTable kJump = make_jump_table();

// s -> M^(2^j) s.  j is uniform across the wave, so the columns come in
// through scalar loads; the per-lane work is a masked XOR per bit.
__device__ inline uint64_t jump_pow2(uint64_t s, int j) {
    const uint32_t lo = static_cast<uint32_t>(s), hi = static_cast<uint32_t>(s >> 32);
    uint64_t r = 0;
#pragma unroll
    for (int b = 0; b < 32; ++b) {
        const uint64_t m = 0 - static_cast<uint64_t>((lo >> b) & 1u);
        r ^= kJump.col[j][b] & m;
    }
#pragma unroll
    for (int b = 0; b < 32; ++b) {
        const uint64_t m = 0 - static_cast<uint64_t>((hi >> b) & 1u);
        r ^= kJump.col[j][32 + b] & m;
    }
    return r;
}

__device__ inline float unit_of(uint64_t draw) {  // next_f32, random.rs:557-564
    return __uint_as_float((static_cast<uint32_t>(draw) & 0x7FFFFFu) | (126u << 23));
}

constexpr float kTwoPiF = 6.28318548202514648438f;  // 2 * std::f32::consts::PI, exact

// next_normal (random.rs:592-615) on the generator state s (advanced twice)
__device__ inline float next_normal(uint64_t &s) {
    s = xs_step(s);
    float u1 = unit_of(s);
    s = xs_step(s);
    const float u2 = unit_of(s);
    if (u1 <= 0.0f) u1 = 1e-7f;
    else if (u1 >= 1.0f) u1 = 1.0f - 1e-7f;
    // f32::ln / f32::cos of the reference: the host libm's logf / cosf,
    // restated (ts_hip_libm.h; 2*pi*u2 is in [0, 2*pi), the range restated)
    const float l = libm::logf_glibc(u1);
    const float r = sqrtf(-2.0f * l);
    const float c = libm::cosf_glibc_small(kTwoPiF * u2);
    const float z = r * c;
    return (__builtin_isnan(z) || __builtin_isinf(z)) ? 0.0f : z;
}

// Thread t owns elements [t << log_run, (t+1) << log_run).  Its first draw
// index is 2 * (t << log_run), so the jump applies M^(2^(j + log_run + 1))
// for each set bit j of t: the wave-uniform high bits of t take scalar
// branches, the six lane bits masked ones.
__global__ __launch_bounds__(kBlock) void randn_kernel(float *__restrict__ out, size_t n,
                                                       uint64_t seed, int log_run, int vec) {
    const int lane = threadIdx.x & 63;
    const uint64_t wave = __builtin_amdgcn_readfirstlane(
        static_cast<uint64_t>(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6));
    uint64_t s = seed;
    const int base = log_run + 1;
    for (int j = 0; j < 6; ++j)
        if ((lane >> j) & 1) s = jump_pow2(s, base + j);
    for (int j = 0; 6 + j + base < 64 && (wave >> j) != 0; ++j)
        if ((wave >> j) & 1) s = jump_pow2(s, base + 6 + j);

    const size_t t = (wave << 6) | static_cast<uint64_t>(lane);
    const size_t run = size_t(1) << log_run;
    const size_t e0 = t << log_run;
    if (e0 >= n) return;
    const size_t e1 = (n - e0 < run) ? n : e0 + run;
    size_t e = e0;
    if (vec) {  // out is 16-byte aligned and runs are multiples of 4 (log_run >= 2)
        for (; e + 4 <= e1; e += 4) {
            float4 q;
            q.x = next_normal(s);
            q.y = next_normal(s);
            q.z = next_normal(s);
            q.w = next_normal(s);
            *reinterpret_cast<float4 *>(out + e) = q;
        }
    }
    for (; e < e1; ++e) out[e] = next_normal(s);
}

// Run length: enough threads to give every SIMD of the device several waves,
// runs of 4 .. 1024 elements (a power of two) so the jump cost (at most 64
// matrix-vector products, about 12 on average) is spread over the run.
static int randn_log_run(size_t n) {
    const size_t want_threads = static_cast<size_t>(device_cu_count()) * 4 * 4 * 64;
    int lr = 2;
    while (lr < 10 && (n >> (lr + 1)) >= want_threads) ++lr;
    return lr;
}

}  // namespace tship

using namespace tship;

extern "C" int ts_hip_randn(float *out, size_t n, uint64_t seed, void *stream) {
    if (n == 0) return TS_HIP_OK;  // random.rs:271-273: empty tensors are left as they are
    if (!out) return TS_HIP_EINVAL;
    // the draw index 2n must fit the 64-bit jump table
    if (n > (size_t(1) << 62)) return TS_HIP_EINVAL;
    const int log_run = randn_log_run(n);
    const size_t threads = (n + (size_t(1) << log_run) - 1) >> log_run;
    const size_t blocks = (threads + kBlock - 1) / kBlock;
    if (blocks > 0x7fffffffULL) return TS_HIP_EINVAL;
    launch(randn_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0,
                       as_stream(stream), out, n, seed, log_run, aligned16(out) ? 1 : 0);
    return launch_status();
}
