// hip_common.h — shared definitions of the gfx950 backend: error checks, wavefront reductions,
// and the device-side storage layouts of the quantized weight formats.
//
// Device weight layouts. A Q4_0 or Q8_0 tensor of nb blocks is stored by this backend as two
// planes inside the same allocation (same total bytes as the GGUF layout):
//     [ qs plane: nb x 16 B (Q4_0) or nb x 32 B (Q8_0) ][ d plane: nb x fp16 ]
// so that a lane's block payload is one (Q4_0) or two (Q8_0) aligned 128-bit loads and a
// wavefront reads consecutive blocks of a row as one contiguous span. Block b of the tensor
// (row-major over rows, then blocks within the row) sits at qs + b*QS and d + b. Q4_K keeps the
// GGUF layout (144-byte blocks are already 16-byte aligned). ggml_backend_tensor_set/get
// translate between layouts, so callers always see GGUF bytes.
//
// Activation ("x") operands of the integer dots are quantized by this backend into:
//     q8 for Q4_0/Q8_0 weights: int8 qs[K], float d[K/32] (the fp16-rounded block scale, as
//         ggml's Q8_0 stores it), int32 s[K/32] (sum of the block's int8 values)
//     q8K for Q4_K weights:    int8 qs[K], float d[K/256], int16 bsums[K/16]
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

#define HIP_CHECK(expr)                                                                             \
    do {                                                                                            \
        hipError_t err_ = (expr);                                                                   \
        if (err_ != hipSuccess) {                                                                   \
            fprintf(stderr, "HIP error %s at %s:%d: %s\n", hipGetErrorName(err_), __FILE__, __LINE__, \
                    hipGetErrorString(err_));                                                       \
            abort();                                                                                \
        }                                                                                           \
    } while (0)

#define HIP_ABORT(...) do { fprintf(stderr, "ggml-hip: " __VA_ARGS__); fputc('\n', stderr); abort(); } while (0)

constexpr int WAVE = 64;

// byte sizes of the device planes
constexpr int Q4_0_QS = 16;
constexpr int Q8_0_QS = 32;
constexpr int Q4_K_BYTES = 144;
constexpr int Q5_K_BYTES = 176;

struct q4k_block { __half d; __half dmin; uint8_t scales[12]; uint8_t qs[128]; };
static_assert(sizeof(q4k_block) == 144, "q4_K block");
// GGUF order: the Q4_K header, the fifth bits (bit j of qh[l]: element l of sub-block j), the nibbles
struct q5k_block { __half d; __half dmin; uint8_t scales[12]; uint8_t qh[32]; uint8_t qs[128]; };
static_assert(sizeof(q5k_block) == 176, "q5_K block");

// DPP lane exchanges (v_mov_dpp): quad_perm xor 1 (0xB1) and xor 2 (0x4E), row_half_mirror (0x141:
// lane i <-> 7 - i within 8 lanes), row_mirror (0x140: i <-> 15 - i within 16). One VALU op each,
// where __shfl_xor goes through ds_bpermute (an LDS round trip). Every lane of the groups involved
// must be active.
template <int CTRL> __device__ __forceinline__ int dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }
template <int CTRL> __device__ __forceinline__ float dpp_f(float v) { return __int_as_float(dpp_i<CTRL>(__float_as_int(v))); }
template <int CTRL> __device__ __forceinline__ double dpp_d(double v) {
    const int lo = dpp_i<CTRL>(__double2loint(v)), hi = dpp_i<CTRL>(__double2hiint(v));
    return __hiloint2double(hi, lo);
}
// the value of v in lane l (uniform)
__device__ __forceinline__ float lane_f(float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); }
// max / sum over aligned groups of 8 lanes (every lane gets the result)
__device__ __forceinline__ float max8_dpp(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    return fmaxf(v, dpp_f<0x141>(v));
}
__device__ __forceinline__ int sum8_dpp(int v) {
    v += dpp_i<0xB1>(v);
    v += dpp_i<0x4E>(v);
    return v + dpp_i<0x141>(v);
}
// sum of a double over the wave: exchanges within each row of 16 lanes, then the four row sums
// added in row order (uniform result)
__device__ __forceinline__ double wave_sum_d_dpp(double v) {
    v += dpp_d<0xB1>(v);
    v += dpp_d<0x4E>(v);
    v += dpp_d<0x141>(v);
    v += dpp_d<0x140>(v);
    const int lo = __double2loint(v), hi = __double2hiint(v);
    double r[4];
#pragma unroll
    for (int k = 0; k < 4; k++) r[k] = __hiloint2double(__builtin_amdgcn_readlane(hi, 16 * k), __builtin_amdgcn_readlane(lo, 16 * k));
    return ((r[0] + r[1]) + r[2]) + r[3];
}

// Whole-wave reductions (every lane active; uniform result). The double sums of the kernels add
// exact quantities (products of F16 values, exps of floats, squares of floats) whose double sum is
// exact in practice, so the pairing does not change them.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

__device__ __forceinline__ double wave_sum_d(double v) { return wave_sum_d_dpp(v); }

// sum / max within aligned groups of G lanes (G a power of two <= 64; every lane gets its group's
// result): DPP within rows of 16 lanes, lane shuffles across rows. The sums add integers held as
// floats, exact in any order.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    if (G >= 2) v += dpp_f<0xB1>(v);
    if (G >= 4) v += dpp_f<0x4E>(v);
    if (G >= 8) v += dpp_f<0x141>(v);
    if (G >= 16) v += dpp_f<0x140>(v);
    if (G >= 32) v += __shfl_xor(v, 16, WAVE);
    if (G >= 64) v += __shfl_xor(v, 32, WAVE);
    return v;
}

template <int G>
__device__ __forceinline__ float group_max(float v) {
    if (G >= 2) v = fmaxf(v, dpp_f<0xB1>(v));
    if (G >= 4) v = fmaxf(v, dpp_f<0x4E>(v));
    if (G >= 8) v = fmaxf(v, dpp_f<0x141>(v));
    if (G >= 16) v = fmaxf(v, dpp_f<0x140>(v));
    if (G >= 32) v = fmaxf(v, __shfl_xor(v, 16, WAVE));
    if (G >= 64) v = fmaxf(v, __shfl_xor(v, 32, WAVE));
    return v;
}

__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// A kernel's arguments sit in device memory that no cache holds when the kernel starts: each scalar
// load of a new 64-byte line of them goes to memory, and the address set-up of a kernel is a chain
// of such loads (an index read from one field selects the next). Measured inside the decode GEMVs:
// about 1 us per link, three to four links before the first weight load went out. Called first in
// a kernel, this reads one dword of every line of its first BYTES bytes of arguments with
// independent loads and waits for them once, so the chain that follows hits the scalar cache.
// Every offset read lies inside the explicit arguments.
typedef const __attribute__((address_space(4))) uint32_t * kernarg_ptr;

template <int BYTES>
__device__ __forceinline__ kernarg_ptr prefetch_kernarg_lines() {
    constexpr int LINES = (BYTES + 63) / 64;
    kernarg_ptr k = (kernarg_ptr) __builtin_amdgcn_kernarg_segment_ptr();
    uint32_t v[LINES + 1];
#pragma unroll
    for (int i = 0; i < LINES; i++) v[i] = k[i * 16];
    v[LINES] = k[(BYTES - 4) / 4];
    // the returned pointer depends on every load: whatever is read through it comes after them
#pragma unroll
    for (int i = 0; i <= LINES; i++) asm volatile("" : "+s"(k) : "s"(v[i]));
    return k;
}

template <int BYTES>
__device__ __forceinline__ void prefetch_kernargs() {
    (void) prefetch_kernarg_lines<BYTES>();
    // nothing is scheduled across this point: the loads above go out first, before any load of
    // the kernel's own and its wait
    __builtin_amdgcn_sched_barrier(0);
}

// For a kernel whose first argument is arg: the prefetch above, and arg read back through a pointer
// that depends on it. The compiler hoists a kernel's argument loads, and the address arithmetic on
// them, above anything that does not feed them; reading the arguments through this reference keeps
// every one of those loads after the prefetch.
template <typename T>
__device__ __forceinline__ const T & kernargs_prefetched(const T & arg) {
    (void) arg;
    return *(const T *) (const __attribute__((address_space(4))) T *) prefetch_kernarg_lines<(int) sizeof(T)>();
}

// Transcendentals of the float ops are evaluated in double and rounded once, i.e. the correctly
// rounded float result (barring astronomically rare double-rounding cases). The CPU oracle defines
// the same semantics, so RoPE angles, softmax weights and SiLU agree bit-for-bit across backends
// instead of drifting by the ulp-level differences of two float libm implementations.
__device__ __forceinline__ float exp_cr(float x) { return (float) exp((double) x); }
__device__ __forceinline__ float cos_cr(float x) { return (float) cos((double) x); }
__device__ __forceinline__ float sin_cr(float x) { return (float) sin((double) x); }
__device__ __forceinline__ float log_cr(float x) { return (float) log((double) x); }
// both of the above from one argument reduction
__device__ __forceinline__ void sincos_cr(float x, float & s, float & c) {
    double sd, cd;
    sincos((double) x, &sd, &cd);
    s = (float) sd;
    c = (float) cd;
}

// MoE routing of one token over at most 256 experts by a workgroup of exactly 256 threads, thread
// t holding the scaled logit w of expert t (-INFINITY for t >= E). The soft_max op's arithmetic:
// the maximum, e = exp(w - max), the sum of the e in double, p = e * (float) (1 / sum); then the
// stable descending order of argsort (ties: the lower expert first) as a rank count over 64-bit
// keys (the bits of p, then 255 - i): finite logits give p in [0, 1], whose bit patterns order as
// the floats do, so rank(i) = the count of keys above expert i's is the count of p[j] > p[i], or
// p[j] == p[i] with j < i. The keys are distinct, so the ranks are too. For E <= 128 two threads
// count an expert's rank over half of the keys each. Leaves p[i] in s_p[i] and the expert of rank
// r < k in s_ids[r] for every thread; every thread must call it. s_key: 256 entries, 16-byte aligned.
__device__ __forceinline__ void moe_route_256(float w, int E, int k, float * s_p, int * s_ids, int * s_cnt,
                                              uint64_t * s_key, float * s_red, double * s_sum) {
    const int t = threadIdx.x;
    float mx = wave_max(fmaxf(-INFINITY, w));
    if ((t % 64) == 0) s_red[t / 64] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    const float v = t < E ? exp_cr(w - mx) : 0.0f;
    double sum = t < E ? (double) v : 0.0;
    sum = wave_sum_d(sum);
    if ((t % 64) == 0) s_sum[t / 64] = sum;
    __syncthreads();
    const float inv = (float) (1.0 / (s_sum[0] + s_sum[1] + s_sum[2] + s_sum[3]));
    const float p = v * inv;
    if (t < E) s_p[t] = p;
    // padding keys (t >= E) are 0: never above another key
    s_key[t] = t < E ? ((uint64_t) __float_as_uint(p) << 32) | (uint32_t) (255 - t) : 0;
    __syncthreads();
    int rank = 0;
    if (E <= 128) {
        const int i = t % 128;
        const uint64_t ki = s_key[i];
        const ulonglong2 * kk = (const ulonglong2 *) (s_key + (t / 128) * 64);
#pragma unroll 8
        for (int q = 0; q < 32; q++) {
            const ulonglong2 u = kk[q];
            rank += (u.x > ki ? 1 : 0) + (u.y > ki ? 1 : 0);
        }
        s_cnt[t] = rank;
        __syncthreads();
        if (t < E) rank = s_cnt[t] + s_cnt[t + 128];
    } else {
        const uint64_t ki = s_key[t];
        const ulonglong2 * kk = (const ulonglong2 *) s_key;
#pragma unroll 8
        for (int q = 0; q < 128; q++) {
            const ulonglong2 u = kk[q];
            rank += (u.x > ki ? 1 : 0) + (u.y > ki ? 1 : 0);
        }
    }
    if (t < E && rank < k) s_ids[rank] = t;
    __syncthreads();
}

// The routing's outputs from moe_route_256's LDS, by one thread: the k expert ids and their
// probabilities divided by their sum (added in rank order in double, rounded to float once:
// the sum_rows and div ops).
__device__ __forceinline__ void moe_route_store(const float * s_p, const int * s_ids, int k, int32_t * ids, float * w) {
    double s = 0.0;
    for (int r = 0; r < k; r++) s += (double) s_p[s_ids[r]];
    const float sf = (float) s;
    for (int r = 0; r < k; r++) {
        ids[r] = s_ids[r];
        w[r] = s_p[s_ids[r]] / sf;
    }
}

// The element index lane t loads: i when below n, else the lane's own first element t (n - 1 for
// the lanes past it). A lane past the end then loads an element that is in bounds and whose value
// is never used (dropped, or stored over that same element's slot with the same value), and most
// lanes of a wave keep distinct addresses that other lanes request anyway, where clamping every
// such lane to n - 1 makes whole waves load one address. Measured on the Q4_0 / Q8_0 GEMV's
// prologue (C2 765.6 -> 771.6 tok/s); the Q4_K kernels' prologues measured faster with the clamp
// (C3 377.3 against 372.0), so they keep it. (A remainder i % n spreads the lanes too, but its
// division before the loads cost more than it saved.)
__device__ __forceinline__ int wrap_index(int i, int n, int t) { return i < n ? i : min(t, n - 1); }

// round half to even, valid for |v| < 2^22 (the result ggml's nearest_int gives)
__device__ __forceinline__ int round_half_even(float v) { return __float2int_rn(v); }

// Pin a float result in a register before a narrowing conversion. Without it the compiler folds
// __float2half_rn(a * b) into one v_fma_mixlo_f16, which rounds the exact product to f16 once
// instead of to float first; the two differ whenever the float product is an f16 rounding tie.
__device__ __forceinline__ float as_f32(float x) {
    asm volatile("" : "+v"(x));
    return x;
}
