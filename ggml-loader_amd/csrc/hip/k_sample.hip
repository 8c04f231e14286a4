// k_sample.hip — token sampling from one row of logits on the device (model.cpp:1675-1728):
// repetition penalty, then argmax (temp <= 0) or temperature, top-k, top-p and the weighted draw of
// std::discrete_distribution, whose uniform variate u the host supplies.
//
// Results are those of the reference's float and double operation chains on the same logits and
// the same u: the exp of each probability is the correctly rounded float exp (the convention of
// every transcendental here), every normalisation divides exactly as written there, and the
// sequential sums (the float sums of the probabilities, the top-p running sum, the double
// accumulate and partial sums of discrete_distribution) run in order on one lane. Equal logits are
// ordered by ascending token id (std::partial_sort leaves their order unspecified).
//
// Fast path (one workgroup, one launch): top-k with k <= SMP_BOUND_K. Each of the 1024 threads
// takes the maximum of its strided share of the row; the k-th largest of those 1024 maxima is a
// lower bound of the k-th largest logit (they are k distinct elements), so every element of the
// top k is among the elements at or above it. Those candidates (normally a few dozen) are
// compacted into LDS, sorted there, and the draw runs on the first k. When the candidates do not
// fit (SMP_MAX_CAND), or k is larger, the host takes the sorted path: a stable device radix sort
// of the whole row (rocPRIM through hipCUB) and the same draw over its first k entries.
#include "hip_common.h"
#include "kernels.h"

#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <climits>

namespace {

constexpr int SMP_THREADS = 1024;
constexpr int SMP_WAVES = SMP_THREADS / WAVE;
constexpr int SMP_FILTER_BITS = 4096;       // direct-mapped filter of penalized ids

static_assert(SMP_BOUND_K <= SMP_THREADS, "one maximum per thread bounds k");
static_assert((SMP_MAX_CAND & (SMP_MAX_CAND - 1)) == 0, "bitonic sort size");

// model.cpp:1679-1686: the penalty applied once per occurrence of the id in the window, in order
__device__ float penalize(float l, int count, float p) {
    for (int j = 0; j < count; j++) l = l > 0.0f ? l / p : l * p;
    return l;
}

// ascending order key of a float; -0 and +0 share a key, NaN takes the key of -inf
__device__ __forceinline__ uint32_t okey(float v) {
    if (v != v) v = -INFINITY;
    const uint32_t b = __float_as_uint(v + 0.0f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float okey_value(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
// candidate key: ascending order is descending value, then ascending id
__device__ __forceinline__ uint64_t ckey(float v, int id) { return ((uint64_t) ~okey(v) << 32) | (uint32_t) id; }
__device__ __forceinline__ float ckey_value(uint64_t c) { return okey_value(~(uint32_t) (c >> 32)); }

// in-place ascending bitonic sort of s[0..n), n a power of two, by the whole workgroup
template <class K>
__device__ void bitonic_sort(K * s, int n) {
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            for (int t = threadIdx.x; t < n / 2; t += SMP_THREADS) {
                const int lo = 2 * stride * (t / stride) + (t % stride);
                const int hi = lo + stride;
                const K a = s[lo], b = s[hi];
                const bool up = (lo & size) == 0;
                if ((a > b) == up) { s[lo] = b; s[hi] = a; }
            }
        }
    }
    __syncthreads();
}

struct draw_smem {
    float x[SMP_CHUNK];     // a chunk of the probability chain's current stage
    float f;                // broadcasts of thread 0
    double d;
    int i;
    int stop;
};

// The draw over the first k values v(0) >= v(1) >= ... (model.cpp:1697-1727 and libstdc++'s
// discrete_distribution: normalise in double, partial sums in order, the last set to 1, then
// lower_bound of u). Stages of the chain are recomputed from v for each pass, chunk by chunk:
//   stage 1: P = exp((v - vmax) / temp)   stage 2: P / sum   stage 3: (P / sum) / s (after top-p)
// Returns (on every thread) the index into the first k, and whether u was used.
template <class V>
__device__ void draw(V v, int k, float temp, float top_p, double u, draw_smem & S, int & idx, int & drew) {
    const int tid = threadIdx.x;
    const float vmax = v(0);
    float sum = 0.0f, s = 0.0f;
    bool renorm = false;
    auto stage = [&](int level, int i) -> float {
        float p = exp_cr((v(i) - vmax) / temp);
        if (level >= 2) p = p / sum;
        if (level >= 3 && renorm) p = p / s;
        return p;
    };
    // run fn(i, x) on thread 0 over i in [0, n) in order; fn returns true to stop
    auto chain = [&](int level, int n, auto fn) {
        for (int c0 = 0; c0 < n; c0 += SMP_CHUNK) {
            const int nc = min(SMP_CHUNK, n - c0);
            for (int i = tid; i < nc; i += SMP_THREADS) S.x[i] = stage(level, c0 + i);
            __syncthreads();
            if (tid == 0) {
                int stop = 0;
                for (int i = 0; i < nc; i++) {
                    if (fn(c0 + i, S.x[i])) { stop = 1; break; }
                }
                S.stop = stop;
            }
            __syncthreads();
            const int stop = S.stop;
            __syncthreads();
            if (stop) break;
        }
    };
    // float sum of the probabilities (model.cpp:1702-1706)
    chain(1, k, [&](int, float x) { sum += x; return false; });
    if (tid == 0) S.f = sum;
    __syncthreads();
    sum = S.f;
    __syncthreads();
    int cutoff = k;
    if (top_p < 1.0f) {
        // running sum up to top_p, then the float sum of the kept ones (model.cpp:1711-1724)
        float cum = 0.0f, s0 = 0.0f;
        if (tid == 0) S.i = k;
        chain(2, k, [&](int i, float x) {
            cum += x;
            if (cum >= top_p) { S.i = i + 1; return true; }
            return false;
        });
        cutoff = S.i;
        chain(2, cutoff, [&](int, float x) { s0 += x; return false; });
        if (tid == 0) S.f = s0;
        __syncthreads();
        s = S.f;
        renorm = true;
        __syncthreads();
    }
    if (cutoff < 2) {
        // discrete_distribution of one weight: index 0, the generator is not called
        idx = 0;
        drew = 0;
        return;
    }
    double sd = 0.0;
    chain(3, cutoff, [&](int, float x) { sd += (double) x; return false; });
    if (tid == 0) S.d = sd;
    __syncthreads();
    sd = S.d;
    __syncthreads();
    double cp = 0.0;
    if (tid == 0) S.i = cutoff - 1;     // the last partial sum is set to 1 > u
    chain(3, cutoff - 1, [&](int i, float x) {
        cp += (double) x / sd;
        if (!(cp < u)) { S.i = i; return true; }
        return false;
    });
    idx = S.i;
    drew = 1;
    __syncthreads();
}

struct sample_smem {
    uint64_t cand[SMP_MAX_CAND];
    uint32_t maxk[SMP_THREADS];
    int pid[SMP_MAX_PEN];
    float pval[SMP_MAX_PEN];
    uint32_t filter[SMP_FILTER_BITS / 32];
    float wv[SMP_WAVES];
    int wi[SMP_WAVES];
    int n_cand;
    draw_smem d;
};

__global__ __launch_bounds__(SMP_THREADS) void sample_kernel(const sample_request a) {
    __shared__ sample_smem S;
    const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE;
    const int n = a.n;

    // penalized ids (sorted ascending by the host) with their penalized logits
    for (int w = tid; w < SMP_FILTER_BITS / 32; w += SMP_THREADS) S.filter[w] = 0;
    __syncthreads();
    for (int j = tid; j < a.n_pen; j += SMP_THREADS) {
        const int id = a.pen_ids[j];
        S.pid[j] = id;
        S.pval[j] = penalize(a.logits[id], a.pen_cnt[j], a.penalty);
        atomicOr(&S.filter[(id % SMP_FILTER_BITS) / 32], 1u << (id % 32));
    }
    if (tid == 0) S.n_cand = 0;
    __syncthreads();
    const int n_pen = a.n_pen;
    auto value = [&](int i) -> float {
        const float raw = a.logits[i];
        if (n_pen && (S.filter[(i % SMP_FILTER_BITS) / 32] >> (i % 32) & 1u)) {
            int lo = 0, hi = n_pen;
            while (lo < hi) {
                const int mid = (lo + hi) / 2;
                if (S.pid[mid] < i) lo = mid + 1; else hi = mid;
            }
            if (lo < n_pen && S.pid[lo] == i) return S.pval[lo];
        }
        return raw;
    };

    if (a.temp <= 0.0f) {
        // model.cpp:1659-1666 on the penalized row: the first index of the maximum; a NaN never
        // replaces the running maximum, and a NaN at index 0 keeps index 0
        float bv = -INFINITY;
        int bi = INT_MAX;
        for (int i = tid; i < n; i += SMP_THREADS) {
            const float v = value(i);
            if (v > bv || (bi == INT_MAX && v == v)) { bv = v; bi = i; }
        }
        for (int o = 1; o < WAVE; o <<= 1) {
            const float ov = __shfl_xor(bv, o, WAVE);
            const int oi = __shfl_xor(bi, o, WAVE);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        if (lane == 0) { S.wv[wave] = bv; S.wi[wave] = bi; }
        __syncthreads();
        if (tid == 0) {
            for (int w = 1; w < SMP_WAVES; w++) {
                if (S.wv[w] > bv || (S.wv[w] == bv && S.wi[w] < bi)) { bv = S.wv[w]; bi = S.wi[w]; }
            }
            const float v0 = value(0);
            a.out[0] = (v0 != v0 || bi == INT_MAX) ? 0 : bi;
            a.out[1] = 0;
            a.out[2] = SMP_OK;
        }
        return;
    }

    const int k = (a.top_k > 0 && a.top_k < n) ? a.top_k : n;
    // lower bound of the k-th largest value: the k-th largest of the threads' maxima (a thread
    // without elements offers -inf, which only lowers the bound)
    uint32_t bound = 0;
    if (k <= SMP_BOUND_K) {
        uint32_t m = okey(-INFINITY);
        for (int i = tid; i < n; i += SMP_THREADS) m = max(m, okey(value(i)));
        S.maxk[tid] = ~m;                       // ascending sort of ~key: descending values
        bitonic_sort(S.maxk, SMP_THREADS);
        bound = ~S.maxk[k - 1];
    }
    // candidates: every element at or above the bound, compacted with one LDS atomic per wave
    for (int base = 0; base < n; base += SMP_THREADS) {
        const int i = base + tid;
        float v = 0.0f;
        bool take = false;
        if (i < n) { v = value(i); take = okey(v) >= bound; }
        const uint64_t mask = __ballot(take);
        const int cnt = __popcll(mask);
        int slot0 = 0;
        if (lane == 0 && cnt) slot0 = atomicAdd(&S.n_cand, cnt);
        slot0 = __shfl(slot0, 0, WAVE);
        const int below = __builtin_amdgcn_mbcnt_hi((uint32_t) (mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t) mask, 0));
        const int slot = slot0 + below;
        if (take && slot < SMP_MAX_CAND) S.cand[slot] = ckey(v, i);
    }
    __syncthreads();
    const int nc = S.n_cand;
    if (nc > SMP_MAX_CAND) {
        if (tid == 0) a.out[2] = SMP_OVERFLOW;
        return;
    }
    int np = 2;
    while (np < nc) np <<= 1;
    for (int i = nc + tid; i < np; i += SMP_THREADS) S.cand[i] = ~(uint64_t) 0;
    bitonic_sort(S.cand, np);
    const float vmax = ckey_value(S.cand[0]);
    if (!isfinite(vmax)) {
        if (tid == 0) a.out[2] = SMP_NONFINITE;
        return;
    }
    int idx, drew;
    draw([&](int i) { return ckey_value(S.cand[i]); }, k, a.temp, a.top_p, a.u, S.d, idx, drew);
    if (tid == 0) {
        a.out[0] = (int) (uint32_t) S.cand[idx];
        a.out[1] = drew;
        a.out[2] = SMP_OK;
    }
}

// ---- sorted path ----------------------------------------------------------------------------

__global__ void sample_keys_kernel(const float * logits, int n, float * keys, int * ids) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    keys[i] = okey_value(okey(logits[i]));     // NaN -> -inf, -0 -> +0
    ids[i] = i;
}

__global__ void sample_pen_kernel(const sample_request a, float * keys) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= a.n_pen) return;
    const int id = a.pen_ids[j];
    keys[id] = okey_value(okey(penalize(a.logits[id], a.pen_cnt[j], a.penalty)));
}

__global__ __launch_bounds__(SMP_THREADS) void sample_sorted_draw_kernel(const sample_request a, const float * keys,
                                                                         const int * ids) {
    __shared__ draw_smem D;
    const int k = (a.top_k > 0 && a.top_k < a.n) ? a.top_k : a.n;
    if (a.temp <= 0.0f) {
        // argmax: the stable sort puts the first index of the maximum first; a NaN at index 0
        // (sorted as -inf) keeps index 0
        if (threadIdx.x == 0) {
            const float l0 = a.logits[0];
            a.out[0] = l0 != l0 ? 0 : ids[0];
            a.out[1] = 0;
            a.out[2] = SMP_OK;
        }
        return;
    }
    if (!isfinite(keys[0])) {
        if (threadIdx.x == 0) a.out[2] = SMP_NONFINITE;
        return;
    }
    int idx, drew;
    draw([&](int i) { return keys[i]; }, k, a.temp, a.top_p, a.u, D, idx, drew);
    if (threadIdx.x == 0) {
        a.out[0] = ids[idx];
        a.out[1] = drew;
        a.out[2] = SMP_OK;
    }
}

size_t cub_sort_bytes(int n) {
    size_t b = 0;
    HIP_CHECK(hipcub::DeviceRadixSort::SortPairsDescending(nullptr, b, (const float *) nullptr, (float *) nullptr,
                                                           (const int *) nullptr, (int *) nullptr, n, 0, 32));
    return b;
}

size_t align256(size_t b) { return (b + 255) & ~(size_t) 255; }

} // namespace

bool sample_fast_path(const sample_request & r) {
    if (r.n_pen > SMP_MAX_PEN) return false;
    if (r.temp <= 0.0f) return true;
    const int k = (r.top_k > 0 && r.top_k < r.n) ? r.top_k : r.n;
    return k <= SMP_BOUND_K || r.n <= SMP_MAX_CAND;
}

void launch_sample(const sample_request & r, hipStream_t st) {
    if (!sample_fast_path(r)) HIP_ABORT("launch_sample: request needs the sorted path");
    sample_kernel<<<1, SMP_THREADS, 0, st>>>(r);
    HIP_CHECK(hipGetLastError());
}

size_t sample_sorted_ws_bytes(int n) {
    return 2 * align256((size_t) n * sizeof(float)) + 2 * align256((size_t) n * sizeof(int)) + align256(cub_sort_bytes(n));
}

void launch_sample_sorted(const sample_request & r, void * ws, size_t ws_bytes, hipStream_t st) {
    if (ws_bytes < sample_sorted_ws_bytes(r.n)) HIP_ABORT("launch_sample_sorted: workspace too small");
    uint8_t * p = (uint8_t *) ws;
    const size_t fb = align256((size_t) r.n * sizeof(float)), ib = align256((size_t) r.n * sizeof(int));
    float * keys = (float *) p;          p += fb;
    float * keys_s = (float *) p;        p += fb;
    int * ids = (int *) p;               p += ib;
    int * ids_s = (int *) p;             p += ib;
    size_t tb = cub_sort_bytes(r.n);
    sample_keys_kernel<<<(r.n + 255) / 256, 256, 0, st>>>(r.logits, r.n, keys, ids);
    HIP_CHECK(hipGetLastError());
    if (r.n_pen > 0) {
        sample_pen_kernel<<<(r.n_pen + 255) / 256, 256, 0, st>>>(r, keys);
        HIP_CHECK(hipGetLastError());
    }
    // stable: equal keys keep ascending ids
    HIP_CHECK(hipcub::DeviceRadixSort::SortPairsDescending(p, tb, keys, keys_s, ids, ids_s, r.n, 0, 32, st));
    sample_sorted_draw_kernel<<<1, SMP_THREADS, 0, st>>>(r, keys_s, ids_s);
    HIP_CHECK(hipGetLastError());
}
