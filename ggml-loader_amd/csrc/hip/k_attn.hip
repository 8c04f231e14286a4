// k_attn.hip — split-KV decode attention over the persistent F16 KV cache (GQA).
//
// Replaces the graph's KQ = K^T Q -> softmax(KQ*scale + mask) -> V^T-materialization -> V KQ
// chain (reference model.cpp:1416-1444) for n_q <= 4 query tokens. Semantics kept from that
// chain: Q is rounded to F16 before the QK dot (ggml converts the F32 operand of an F16 mul_mat),
// scores are scaled, masked, and softmax-normalized in f32; V is never transposed or copied.
//
// Pass 1 (grid: splits x kv_heads): one wavefront per (chunk of 64 positions, KV head). The
// chunk's K rows are staged through LDS (coalesced 16-byte loads; rows padded to 65 dwords so
// lane t reading row t is conflict-free); lane t then computes the scores of position t for every
// query head of the GQA group with packed f16 dot products (v_dot2_f32_f16). The chunk's max
// and exp-sum per head come from wave reductions; the V rows are streamed once (coalesced, two
// dims per lane) into an unnormalized accumulator per head. Partials (max, sum, acc[hd]) go to
// scratch. Pass 2 (grid: heads x queries) merges the splits with the usual max-rescaling and
// writes the output, optionally also as Q8_0 blocks for the output projection.
#include "kernels.h"

#include "ggml.h"

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int ATT_CHUNK = 64;
constexpr int ATT_MAX_Q = 4;

int64_t attn_scratch_bytes(int n_kv, int n_q, int n_head, int hd) {
    const int64_t splits = (n_kv + ATT_CHUNK - 1) / ATT_CHUNK;
    return splits * (int64_t) n_head * n_q * (hd + 2) * (int64_t) sizeof(float);
}

__device__ __forceinline__ float mask_at(const attn_launch & A, int q, int t) {
    if (!A.mask) return 0.0f;
    const char * row = (const char *) A.mask + (int64_t) q * A.mask_nb1;
    return A.mask_f16 ? __half2float(((const __half *) row)[t]) : ((const float *) row)[t];
}

template <int HD, int G>
__global__ __launch_bounds__(64) void attn_split_kernel(const attn_launch A) {
    constexpr int HD2 = HD / 2;          // half2 per row
    constexpr int STRIDE = HD2 + 1;      // padded LDS row (dwords)
    __shared__ uint32_t s_k[ATT_CHUNK * STRIDE];
    __shared__ uint32_t s_q[ATT_MAX_Q][G][HD2];
    __shared__ float s_p[ATT_MAX_Q][G][ATT_CHUNK];

    const int split = blockIdx.x;
    const int kvh = blockIdx.y;
    const int lane = threadIdx.x;
    const int t0 = split * ATT_CHUNK;
    const int nt = min(ATT_CHUNK, A.n_kv - t0);
    const int n_q = A.n_q;

    // stage this chunk's K rows (16-byte pieces, 4 rows x 16 pieces per wave-wide load at HD=128)
    constexpr int PIECES = HD / 8; // 8 halves per 16-byte piece
    for (int pc = lane; pc < ATT_CHUNK * PIECES; pc += 64) {
        const int r = pc / PIECES, c = pc % PIECES;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (r < nt) v = *(const uint4 *) (A.k + (int64_t) kvh * A.k_nb1 + (int64_t) (t0 + r) * A.k_nb2 + c * 8);
        uint32_t * dst = s_k + r * STRIDE + c * 4;
        dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
    }
    // queries of this KV head's group, rounded to f16
    for (int i = lane; i < n_q * G * HD2; i += 64) {
        const int q = i / (G * HD2), g = (i / HD2) % G, d2 = i % HD2;
        const int h = kvh * G + g;
        const float * qp = A.q + (int64_t) h * A.q_nb1 + (int64_t) q * A.q_nb2 + 2 * d2;
        const __half2 hv = __floats2half2_rn(qp[0], qp[1]);
        s_q[q][g][d2] = *(const uint32_t *) &hv;
    }
    __syncthreads();

    float m_loc[ATT_MAX_Q][G];
    float l_loc[ATT_MAX_Q][G];
#pragma unroll
    for (int q = 0; q < ATT_MAX_Q; q++) {
        if (q >= n_q) break;
        float sc[G];
#pragma unroll
        for (int g = 0; g < G; g++) sc[g] = 0.0f;
        if (lane < nt) {
            const uint32_t * kr = s_k + lane * STRIDE;
#pragma unroll 8
            for (int d2 = 0; d2 < HD2; d2++) {
                const uint32_t kk = kr[d2];
                const f16x2 kv = __builtin_bit_cast(f16x2, kk);
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const f16x2 qv = __builtin_bit_cast(f16x2, s_q[q][g][d2]);
                    sc[g] = __builtin_amdgcn_fdot2(kv, qv, sc[g], false);
                }
            }
        }
        const float mv = lane < nt ? mask_at(A, q, t0 + lane) : -INFINITY;
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float s = lane < nt ? sc[g] * A.scale + mv : -INFINITY;
            const float m = wave_max(s);
            const float p = (m == -INFINITY) ? 0.0f : expf(s - m);
            const float l = wave_sum(p);
            m_loc[q][g] = m;
            l_loc[q][g] = l;
            s_p[q][g][lane] = p;
        }
    }
    __syncthreads();

    // V: lane owns dims (2*lane, 2*lane+1); unnormalized sum of p * v over the chunk
    const bool has_dim = 2 * lane < HD;
    float acc[ATT_MAX_Q][G][2];
    for (int q = 0; q < ATT_MAX_Q; q++)
#pragma unroll
        for (int g = 0; g < G; g++) { acc[q][g][0] = 0.0f; acc[q][g][1] = 0.0f; }
    if (has_dim) {
        const __half2 * vb = (const __half2 *) (A.v + (int64_t) kvh * A.v_nb1) + lane;
#pragma unroll 4
        for (int t = 0; t < nt; t++) {
            const float2 vf = __half22float2(vb[(int64_t) (t0 + t) * (A.v_nb2 / 2)]);
#pragma unroll
            for (int q = 0; q < ATT_MAX_Q; q++) {
                if (q >= n_q) break;
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const float p = s_p[q][g][t];
                    acc[q][g][0] += p * vf.x;
                    acc[q][g][1] += p * vf.y;
                }
            }
        }
    }
    // partial layout: [split][q][head] x (max, sum, acc[HD])
#pragma unroll
    for (int q = 0; q < ATT_MAX_Q; q++) {
        if (q >= n_q) break;
#pragma unroll
        for (int g = 0; g < G; g++) {
            const int h = kvh * G + g;
            float * part = A.scratch + (((int64_t) split * n_q + q) * A.n_head + h) * (HD + 2);
            if (lane == 0) { part[0] = m_loc[q][g]; part[1] = l_loc[q][g]; }
            if (has_dim) { part[2 + 2 * lane] = acc[q][g][0]; part[3 + 2 * lane] = acc[q][g][1]; }
        }
    }
}

// merge the splits of one (head, query); block = HD threads (one per dim)
template <int HD>
__global__ void attn_combine_kernel(const attn_launch A, int n_splits) {
    const int h = blockIdx.x, q = blockIdx.y, d = threadIdx.x;
    float m = -INFINITY;
    for (int s = 0; s < n_splits; s++) {
        const float * part = A.scratch + (((int64_t) s * A.n_q + q) * A.n_head + h) * (HD + 2);
        m = fmaxf(m, part[0]);
    }
    float l = 0.0f, o = 0.0f;
    if (m != -INFINITY) {
        for (int s = 0; s < n_splits; s++) {
            const float * part = A.scratch + (((int64_t) s * A.n_q + q) * A.n_head + h) * (HD + 2);
            if (part[0] == -INFINITY) continue;
            const float w = expf(part[0] - m);
            l += w * part[1];
            o += w * part[2 + d];
        }
    }
    const float v = l > 0.0f ? o / l : 0.0f;
    const int64_t oi = (int64_t) h * HD + d;
    A.out[(int64_t) q * A.out_nb1 + oi] = v;
    if (A.out_q.qs) {
        // Q8_0 blocks of 32 consecutive dims (HD % 32 == 0): lanes d..d+31 share a half-wave
        const float amax = group_max<32>(fabsf(v));
        const float dd = amax / 127;
        const float id = dd ? 1.0f / dd : 0.0f;
        const int qv = (int) roundf(v * id);
        const float qsum = group_sum<32>((float) qv);
        const int64_t K = (int64_t) A.n_head * HD;
        A.out_q.qs[q * K + oi] = (int8_t) qv;
        if ((d % 32) == 0) {
            A.out_q.d[q * (K / 32) + oi / 32] = __half2float(__float2half_rn(dd));
            A.out_q.s[q * (K / 32) + oi / 32] = (int32_t) qsum;
        }
    }
}

template <int HD, int G>
static void launch_attn_t(const attn_launch & A, hipStream_t st) {
    const int splits = (A.n_kv + ATT_CHUNK - 1) / ATT_CHUNK;
    hipLaunchKernelGGL((attn_split_kernel<HD, G>), dim3(splits, A.n_head_kv), dim3(64), 0, st, A);
    HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(attn_combine_kernel<HD>, dim3(A.n_head, A.n_q), dim3(HD), 0, st, A, splits);
    HIP_CHECK(hipGetLastError());
}

template <int HD>
static void launch_attn_hd(const attn_launch & A, hipStream_t st) {
    const int G = A.n_head / A.n_head_kv;
    switch (G) {
        case 1: launch_attn_t<HD, 1>(A, st); break;
        case 2: launch_attn_t<HD, 2>(A, st); break;
        case 3: launch_attn_t<HD, 3>(A, st); break;
        case 4: launch_attn_t<HD, 4>(A, st); break;
        case 5: launch_attn_t<HD, 5>(A, st); break;
        case 6: launch_attn_t<HD, 6>(A, st); break;
        case 7: launch_attn_t<HD, 7>(A, st); break;
        case 8: launch_attn_t<HD, 8>(A, st); break;
        default: HIP_ABORT("attn: unsupported GQA group %d", G);
    }
}

void launch_attn_decode(const attn_launch & A, hipStream_t st) {
    if (A.n_q < 1 || A.n_q > ATT_MAX_Q) HIP_ABORT("attn: n_q %d out of range", A.n_q);
    if (A.n_head % A.n_head_kv) HIP_ABORT("attn: n_head %% n_head_kv");
    if (A.scratch_bytes < attn_scratch_bytes(A.n_kv, A.n_q, A.n_head, A.hd)) HIP_ABORT("attn: scratch too small");
    if (A.out_q.qs && (A.hd % 32)) HIP_ABORT("attn: quantized output needs hd %% 32 == 0");
    switch (A.hd) {
        case 64: launch_attn_hd<64>(A, st); break;
        case 96: launch_attn_hd<96>(A, st); break;
        case 128: launch_attn_hd<128>(A, st); break;
        default: HIP_ABORT("attn: unsupported head dim %d", A.hd);
    }
}
