// k_attn.hip — split-KV decode attention over the persistent F16 KV cache (GQA).
//
// Replaces the graph's KQ = K^T Q -> softmax(KQ*scale + mask) -> V^T-materialization -> V KQ
// chain (reference model.cpp:1416-1444) for n_q <= 4 query tokens, with that chain's arithmetic:
//   * QK dot: Q rounded to F16 (ggml converts the F32 operand of an F16 mul_mat), products of the
//     two F16 values (exact in f32) summed in double, the sum rounded to float once;
//   * softmax over the whole row: w = kq*scale + mask, M = max w, e = exp(w - M), S = sum e in
//     double, p = e * (float)(1/S), then p rounded to F16 (the operand conversion of the V mul_mat;
//     flash_attn_ext, which has no such operand, keeps p a float: attn_launch::p_f32);
//   * PV: products of F16 p and F16 V (exact in f32) summed in double, rounded to float once.
// The double sums are exact for these operands in practice, so the result does not depend on the
// summation order and equals the CPU reference's float. V is read in place (never transposed).
// This matters beyond the op: the attention output is quantized to Q8_0 for the output
// projection, and any drift shifts values across int8 rounding boundaries, which the following
// layers amplify.
//
// Four launches (three for one query over at most PV_FS_MAX_KV positions), each issuing its memory
// reads in independent batches (a dependent load per loop iteration would put one L2/HBM round
// trip per iteration on the critical path):
//   scores   (64-position chunk, KV head) workgroups: the chunk's K rows staged through LDS with
//            coalesced 16-byte loads (rows padded by one dword so lane t reading row t is
//            conflict-free); one wave per (query, head of the GQA group), lane = position; each
//            row's chunk maximum.
//   stats    (query, head, 1024-position segment) workgroups: M = the maximum of the row's chunk
//            maxima, e = exp(s - M) written over each score, the segment's sum of e in double.
//   pv       (128-position chunk, KV head) workgroups: 1/S from the segment sums (added in segment
//            order), p = F16(e * (1/S)) for the chunk, the chunk's V rows staged in LDS (every load
//            issued up front), one partial per (chunk, query, head) accumulated in double; one wave
//            per (query, head), two dims per lane. For one query over a short row, (chunk, head)
//            workgroups that form M, e and S themselves, and no stats launch.
//   combine  one thread per output element: the partials added in chunk order (+ Q8_0 blocks).
// Workgroups exchange results only across launch boundaries: a flag-and-fence hand-off inside a
// launch costs a write-back and invalidation of the L2 of every XCD that takes part (measured: the
// combine folded into the PV launch behind a last-workgroup count took it from 8.6 to 44 us).
// Scratch: see attn_scratch.
#include "kernels.h"
#include "tview_ops.h"

#include "ggml.h"

#include <type_traits>

constexpr int ATT_CHUNK = 64;
constexpr int ATT_MAX_Q = 4;
constexpr int ATT_THREADS = 256;
constexpr int ATT_WAVES = ATT_THREADS / WAVE;

constexpr int PV_CHUNK = 128;
constexpr int STATS_PER_THREAD = 4;                          // scores per thread of a statistics workgroup
constexpr int STATS_SEG = ATT_THREADS * STATS_PER_THREAD;    // positions per statistics workgroup

__host__ __device__ inline int attn_chunks(int n_kv) { return (n_kv + ATT_CHUNK - 1) / ATT_CHUNK; }
__host__ __device__ inline int attn_segs(int n_kv) { return (n_kv + STATS_SEG - 1) / STATS_SEG; }

// Scratch (all per row = (query, head)): scores f32 [n_kv] (after the statistics launch: e =
// exp(s - M), M the row maximum), the maximum of each 64-position chunk f32 [chunks], the sum of e
// over each statistics segment f64 [segs], and the PV partials f64 [pv chunks][n_q][n_head][hd].
struct attn_scratch {
    float * scores;
    float * cmax;
    double * ssum;
    double * parts;
};

__host__ __device__ inline attn_scratch scratch_of(const attn_launch & A) {
    const int64_t nrow = (int64_t) A.n_q * A.n_head;
    attn_scratch s;
    s.scores = A.scratch;
    s.cmax = s.scores + nrow * A.n_kv;
    const int64_t nf = nrow * A.n_kv + nrow * attn_chunks(A.n_kv);
    s.ssum = (double *) (A.scratch + nf + (nf & 1));
    s.parts = s.ssum + nrow * attn_segs(A.n_kv);
    return s;
}

// Row r of a chunk of nt rows at position t0 for a load whose value past the chunk's end is not
// used: r itself, else the same row of the previous chunk (in bounds, and a distinct address per
// lane) or, in the first chunk, its last row. Clamping every lane past the end to row nt - 1 would
// make them all load one row: the last chunk of a row of 2^k + 1 positions holds one.
__device__ __forceinline__ int tail_row(int r, int nt, int t0, int chunk) { return r < nt ? r : t0 >= chunk ? r - chunk : nt - 1; }

int64_t attn_scratch_bytes(int n_kv, int n_q, int n_head, int hd) {
    const int64_t nrow = (int64_t) n_q * n_head;
    const int64_t nf = nrow * n_kv + nrow * attn_chunks(n_kv);
    const int64_t pv_chunks = (n_kv + PV_CHUNK - 1) / PV_CHUNK;
    return (nf + (nf & 1)) * (int64_t) sizeof(float) +
           (nrow * attn_segs(n_kv) + pv_chunks * nrow * hd) * (int64_t) sizeof(double);
}

// r / g for 0 <= r < DIV_SMALL_MAX and 1 <= g <= 64, with inv_g = 1.0f / g, in three float
// operations: (r + 0.5) / g lies at least 1 / (2 g) >= 1/128 from every integer, and the float
// product is within DIV_SMALL_MAX * 2^-23 = 1/512 of it, so truncating it gives the quotient.
constexpr int DIV_SMALL_MAX = 16384;
__device__ __forceinline__ int div_small(int r, float inv_g) { return (int) (((float) r + 0.5f) * inv_g); }

__device__ __forceinline__ float mask_at(const attn_launch & A, int q, int t) {
    if (!A.mask) return 0.0f;
    const char * row = (const char *) A.mask + (int64_t) q * A.mask_nb1;
    return A.mask_f16 ? __half2float(((const __half *) row)[t]) : ((const float *) row)[t];
}

// Dynamic LDS of the scores kernel, sized for the launch's n_q new tokens (in floats): the Q rows
// as the dots read them, as doubles [n_q * G][HD + 8] (each quarter of a row padded by two doubles,
// so that the four quarters the lanes of a quad read start in different banks), the Q source rows [n_q * G][HD], the new K and V source
// rows [n_q][HD] each, the norm weights of Q and K [HD] each, the chunk's mask rows
// [n_q][ATT_CHUNK], the (cos, sin) pairs [n_q][HD / 2] and the norm scales [n_q * G + n_q].
template <int HD, int G>
__host__ __device__ constexpr int scores_dyn_floats(int n_q) {
    return 2 * n_q * G * (HD + 8) + n_q * G * HD + 2 * n_q * HD + 2 * HD + n_q * ATT_CHUNK + n_q * HD + n_q * G + n_q;
}

// Register budget: four waves per SIMD, so that four workgroups of a long row share each CU.
template <int HD, int G>
__global__ __launch_bounds__(ATT_THREADS, 4) void attn_scores_kernel(const attn_launch A_) {
    const attn_launch & A = kernargs_prefetched(A_);
    constexpr int HD2 = HD / 2;
    constexpr int STRIDE = HD2 + 4;   // dwords per staged K row: 16-byte aligned, rows offset by 4 banks
    __shared__ __align__(16) uint32_t s_k[ATT_CHUNK * STRIDE];
    __shared__ __align__(16) uint32_t s_knew[ATT_MAX_Q * HD2];   // the new tokens' rotated K rows (F16)
    __shared__ float s_cm[ATT_WAVES][ATT_MAX_Q * 8];
    extern __shared__ __align__(16) float s_dyn[];
    // blockIdx.y: a group of G consecutive heads (all heads of KV head kvh, or a part of them when
    // the launch splits a large GQA group over several workgroups); h0 its first head
    const int split = blockIdx.x, h0 = blockIdx.y * G;
    const int kvh = __builtin_amdgcn_readfirstlane(div_small(h0, A.s_inv_gqa));
    const bool kv_writer = h0 == kvh * A.s_gqa;   // the first group of a KV head appends K and V
    const int t = threadIdx.x, lane = t % WAVE, wave = t / WAVE;
    const int t0 = split * ATT_CHUNK;
    const int nt = min(ATT_CHUNK, A.n_kv - t0);
    const int q0 = blockIdx.z * ATT_MAX_Q;            // this workgroup's queries: q0 .. q0 + n_q - 1
    const int n_q = min(ATT_MAX_Q, A.n_q - q0);
    const attn_scratch S = scratch_of(A);
    constexpr int DQ = HD / 4;                        // head dims per quarter (per lane in the dots)
    constexpr int QRS = 4 * (DQ + 2);                 // doubles per staged Q row
    double * s_qr = (double *) s_dyn;                 // [n_q * G][QRS]
    float * s_q = (float *) (s_qr + n_q * G * QRS);   // [n_q * G][HD]
    float * s_kx = s_q + n_q * G * HD;                // [n_q][HD]
    float * s_vx = s_kx + n_q * HD;                   // [n_q][HD]
    float * s_qw = s_vx + n_q * HD;                   // [HD]
    float * s_kw = s_qw + HD;                         // [HD]
    float * s_mk = s_kw + HD;                         // [n_q][ATT_CHUNK]
    float2 * s_cs = (float2 *) (s_mk + n_q * ATT_CHUNK);   // [n_q][HD / 2]
    float * s_qs = (float *) (s_cs + n_q * HD2);      // [n_q * G]
    float * s_ks = s_qs + n_q * G;                    // [n_q]

    // Everything else this workgroup reads goes out before the chunk's K loads, so that waiting for
    // it never waits for them (loads complete in issue order): the Q source rows (before QK-Norm and
    // RoPE), the new tokens' K and V source rows, norm weights and positions (RoPE), the chunk's
    // mask values. Indices are clamped and the loads unconditional; values past the ends are never
    // used. Without RoPE the K / V / weight / position loads read Q again (valid, unused).
    // (Source rows and strides as resolved by launch_attn_decode; each load's offset is a 32-bit
    // per-lane part over a base that is uniform across the workgroup.)
    constexpr int QR = (ATT_MAX_Q * G * HD + ATT_THREADS - 1) / ATT_THREADS;
    constexpr int KR = (ATT_MAX_Q * HD + ATT_THREADS - 1) / ATT_THREADS;
    const bool qnorm = A.rope && A.qn.x, knorm = A.rope && A.kn.x;
    const int nqe = n_q * G * HD, nke = n_q * HD;
    float qv[QR], kx[KR], vx[KR];
    {
        // (unsigned indices: quotients by constants are shifts and multiplies)
        const float * qb = A.sq + (h0 * A.sq1 + q0 * A.sq2);
#pragma unroll
        for (int j = 0; j < QR; j++) {
            const unsigned i = (unsigned) min(t + j * ATT_THREADS, nqe - 1);
            const unsigned pr = i / HD;
            qv[j] = qb[(pr % G) * A.sq1 + (pr / G) * A.sq2 + i % HD];
        }
        const float * kb = A.sk + kvh * A.sk1, * vb = A.sv + kvh * A.sv1;
#pragma unroll
        for (int j = 0; j < KR; j++) {
            const unsigned i = (unsigned) min(t + j * ATT_THREADS, nke - 1);
            kx[j] = kb[(i / HD) * A.sk2 + i % HD];
            vx[j] = vb[(i / HD) * A.sv2 + i % HD];
        }
    }
    const float qw = A.sqw[min(t, HD - 1)];
    const float kw = A.skw[min(t, HD - 1)];
    const int half = A.s_half;
    const int tp = min(t, n_q * half - 1);          // this thread's rotation pair (clamped)
    const int tq = (tp >= half) + (tp >= 2 * half) + (tp >= 3 * half);   // its token (n_q <= 4 with RoPE)
    static_assert(ATT_MAX_Q == 4, "the token of a rotation pair");
    const int32_t my_pos = A.spos[tq];
    const bool cs_read = A.rope && A.cs_mode == 2;
    const float2 cs_in = (cs_read ? A.cs_tab : (const float2 *) A.sq)[cs_read ? tp : 0];
    // the chunk's mask values (0 without a mask): an F32 and an F16 load per query, both
    // unconditional (the one of the other type reads Q), so that the dots below load nothing
    const bool mask32 = A.mask && !A.mask_f16, mask16 = A.mask && A.mask_f16;
    const int mbase = q0 * A.s_mask_stride + t0;
    const float * mrow32 = (const float *) (mask32 ? A.mask : (const void *) A.sq) + (mask32 ? mbase : 0);
    const __half * mrow16 = (const __half *) (mask16 ? A.mask : (const void *) A.sq) + (mask16 ? mbase : 0);
    // (raw values here, converted after the K loads are out: a conversion here would wait for
    // every load issued so far)
    float m32[ATT_MAX_Q];
    __half m16[ATT_MAX_Q];
    {
        const int lt = min(lane, nt - 1);
#pragma unroll
        for (int q = 0; q < ATT_MAX_Q; q++) {
            const int mo = min(q, n_q - 1) * A.s_mask_stride + lt;
            m32[q] = mrow32[mask32 ? mo : 0];
            m16[q] = mrow16[mask16 ? mo : 0];
        }
    }

    // The chunk's K rows (16-byte pieces; every load unconditional, at a clamped row, since a
    // guarded load makes the compiler wait for all loads before the next one) stay in registers
    // while everything else happens: the loaded values into LDS and the (cos, sin) of every rotation pair of the new
    // tokens (one pair per thread; Q and K rotate with the same positions and parameters), then
    // QK-Norm and RoPE. Only then are the K rows stored to LDS, which waits for them. The stores
    // are unconditional, at the clamped indices (a thread past the end stores the last value
    // again): a guarded store would let the compiler move its load behind the K loads.
    constexpr int PIECES = HD / 8;                                   // 16-byte pieces per K row
    constexpr int KITER = ATT_CHUNK * PIECES / ATT_THREADS;
    uint4 kv[KITER];
    {
        const __half * kbase = A.k + kvh * A.k_nb1 + t0 * A.k_nb2;
#pragma unroll
        for (int it = 0; it < KITER; it++) {
            const unsigned pc = t + it * ATT_THREADS;
            const unsigned r = pc / PIECES, c = pc % PIECES;
            kv[it] = *(const uint4 *) (kbase + (tail_row((int) r, nt, t0, ATT_CHUNK) * A.k_s2 + (int) c * 8));
        }
    }
    __builtin_amdgcn_sched_barrier(0);   // every load above is out before any wait
    float mk[ATT_MAX_Q];
#pragma unroll
    for (int q = 0; q < ATT_MAX_Q; q++) mk[q] = mask32 ? m32[q] : mask16 ? __half2float(m16[q]) : 0.0f;
#pragma unroll
    for (int j = 0; j < QR; j++) s_q[min(t + j * ATT_THREADS, nqe - 1)] = qv[j];
#pragma unroll
    for (int j = 0; j < KR; j++) {
        const int i = min(t + j * ATT_THREADS, nke - 1);
        s_kx[i] = kx[j];
        s_vx[i] = vx[j];
    }
    s_qw[min(t, HD - 1)] = qw;
    s_kw[min(t, HD - 1)] = kw;
#pragma unroll
    for (int q = 0; q < ATT_MAX_Q; q++) s_mk[min(q, n_q - 1) * ATT_CHUNK + min(lane, nt - 1)] = mk[q];
    {
        float c = 1.0f, sn = 0.0f;
        if (cs_read) {
            c = cs_in.x;
            sn = cs_in.y;
        } else if (A.rope) {
            rope_pair_cs(A.rq.p, A.rq.ff, my_pos, tp - tq * half, c, sn);
            if (A.cs_mode == 1 && blockIdx.x == 0 && blockIdx.y == 0 && t < n_q * half) A.cs_tab[tp] = make_float2(c, sn);
        }
        s_cs[tp] = make_float2(c, sn);
    }
    __syncthreads();   // source rows, weights, mask, (cos, sin) in LDS (the K rows may still be loading)

    // QK-Norm folded in: the scale of each Q row of the group and of each new K row, one wave per
    // row (the sum of squares in double, as the rms_norm op)
    if (qnorm || knorm) {
        const int nrq = qnorm ? n_q * G : 0, nr = nrq + (knorm ? n_q : 0);
        for (int r = wave; r < nr; r += ATT_WAVES) {
            const bool isq = r < nrq;
            const float * xr = isq ? s_q + r * HD : s_kx + (r - nrq) * HD;
            double ss = 0.0;
            for (int e = lane; e < HD; e += WAVE) {
                const float v = xr[e];
                ss += (double) (v * v);
            }
            ss = wave_sum_d(ss);
            if (lane == 0) {
                const float sc = 1.0f / sqrtf((float) (ss / (double) HD) + (isq ? A.qn.eps : A.kn.eps));
                if (isq) s_qs[r] = sc;
                else s_ks[r - nrq] = sc;
            }
        }
        __syncthreads();
    }
    // the Q rows as the dots read them: [normalized,] rotated, rounded to F16 (the mul_mat's
    // conversion of Q). One rotation pair, or one element past n_dims, per item.
    const int np = A.rope ? A.rq.p.n_dims / 2 : 0;
    const bool neox = (A.rq.p.mode & GGML_ROPE_TYPE_NEOX) != 0;
    const int per_row = HD - np;
    for (int i = t; i < n_q * G * per_row; i += ATT_THREADS) {
        const int pr = i / per_row, k = i % per_row;
        const float * xr = s_q + pr * HD;
        double * yr = s_qr + pr * QRS;
        auto qr_at = [](int d) { return d / DQ * (DQ + 2) + d % DQ; };
        const float sc = qnorm ? s_qs[pr] : 1.0f;
        if (k < np) {
            const int a0 = neox ? k : 2 * k, a1 = neox ? k + np : 2 * k + 1;
            float x0 = xr[a0], x1 = xr[a1];
            if (qnorm) {
                x0 = (x0 * sc) * s_qw[a0];
                x1 = (x1 * sc) * s_qw[a1];
            }
            const float2 cs = s_cs[(pr / G) * np + k];
            yr[qr_at(a0)] = (double) __half2float(__float2half_rn(as_f32(x0 * cs.x - x1 * cs.y)));
            yr[qr_at(a1)] = (double) __half2float(__float2half_rn(as_f32(x0 * cs.y + x1 * cs.x)));
        } else {
            const int d = 2 * np + (k - np);
            float v = xr[d];
            if (qnorm) v = (v * sc) * s_qw[d];
            yr[qr_at(d)] = (double) __half2float(__float2half_rn(as_f32(v)));
        }
    }
    // the new positions of this chunk: K rotated into the cache (by the workgroup of the KV head's
    // first head group) and into s_knew, which the dots read for these positions; V appended
    const int first_new = A.n_kv - n_q;
    const bool has_new = A.rope && first_new + n_q > t0 && first_new < t0 + nt;
    if (has_new) {
        for (int i = t; i < nke; i += ATT_THREADS) {
            const int tk = i / HD, d = i % HD;
            const int pos = first_new + tk;
            if (pos < t0 || pos >= t0 + nt) continue;
            const float * xr = s_kx + tk * HD;
            const float sc = knorm ? s_ks[tk] : 1.0f;
            const float kr = rope_value_with(A.rk.p, d, s_cs + tk * np, [&](int e) {
                return knorm ? (xr[e] * sc) * s_kw[e] : xr[e];
            });
            if (kv_writer) {
                st(at(A.rk.dst, d, kvh, tk, 0), GGML_TYPE_F16, kr);
                st(at(A.rv.dst, d, kvh, tk, 0), GGML_TYPE_F16, s_vx[i]);
            }
            ((__half *) (s_knew + tk * HD2))[d] = __float2half_rn(as_f32(kr));
        }
    }
    asm volatile("" ::: "memory");   // the K rows' LDS stores (and their wait) stay after the above
#pragma unroll
    for (int it = 0; it < KITER; it++) {
        const int pc = t + it * ATT_THREADS;
        const int r = pc / PIECES, c = pc % PIECES;
        const bool live = r < nt;            // rows past the end: zero (their loads read the last row)
        uint32_t * d = s_k + r * STRIDE + c * 4;
        d[0] = live ? kv[it].x : 0u; d[1] = live ? kv[it].y : 0u; d[2] = live ? kv[it].z : 0u; d[3] = live ? kv[it].w : 0u;
    }
    __syncthreads();

    // ---- dots: wave w takes positions 16w .. 16w + 15 of the chunk; lane = (position, quarter of
    // the head dims). The lane's K slice is widened to double once and kept in registers for every
    // (query, head) row of the group. Each product of two F16 values is exact in double, so
    // fma(k, q, acc) rounds as acc + (double) (k * q) does: the sum accumulates in double (exact for
    // these operands, so splitting it over chains and quarters does not change it), then the four
    // quarters are added by DPP within each quad of lanes. ----
    const int pi = lane / 4, dq = lane % 4;
    const int tl = wave * 16 + pi;                      // position in the chunk
    const bool ok = tl < nt;
    double kd[DQ];
    {
        const bool is_new = has_new && ok && t0 + tl >= first_new;
        const uint32_t * src = is_new ? s_knew + (t0 + tl - first_new) * HD2 : s_k + tl * STRIDE;
        const uint4 * kp = (const uint4 *) (src + dq * (DQ / 2));
#pragma unroll
        for (int j = 0; j < DQ / 8; j++) {
            const uint4 v = kp[j];
            const uint32_t w[4] = { v.x, v.y, v.z, v.w };
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float2 f = __half22float2(*(const __half2 *) &w[e]);
                kd[8 * j + 2 * e] = (double) f.x;
                kd[8 * j + 2 * e + 1] = (double) f.y;
            }
        }
    }
    for (int pr = 0; pr < n_q * G; pr++) {
        const int q = pr / G, h = h0 + pr % G;
        const double2 * qv2 = (const double2 *) (s_qr + pr * QRS + dq * (DQ + 2));
        double a[4] = { 0.0, 0.0, 0.0, 0.0 };
#pragma unroll
        for (int j = 0; j < DQ / 4; j++) {
            const double2 qa = qv2[2 * j], qb2 = qv2[2 * j + 1];
            a[0] = fma(kd[4 * j], qa.x, a[0]);
            a[1] = fma(kd[4 * j + 1], qa.y, a[1]);
            a[2] = fma(kd[4 * j + 2], qb2.x, a[2]);
            a[3] = fma(kd[4 * j + 3], qb2.y, a[3]);
        }
        double dot = (a[0] + a[1]) + (a[2] + a[3]);
        dot += dpp_d<0xB1>(dot);
        dot += dpp_d<0x4E>(dot);
        // softmax input as the graph forms it: (float) kq * scale + mask
        float sv = -INFINITY;
        if (ok) {
            const float mv = s_mk[q * ATT_CHUNK + tl];
            sv = mv == -INFINITY ? -INFINITY : (float) dot * A.scale + mv;
            if (dq == 0) S.scores[((int64_t) (q0 + q) * A.n_head + h) * A.n_kv + t0 + tl] = sv;
        }
        // the row's maximum over this wave's 16 positions (every lane of a quad holds its value)
        sv = fmaxf(sv, dpp_f<0x141>(sv));
        sv = fmaxf(sv, dpp_f<0x140>(sv));
        sv = fmaxf(fmaxf(lane_f(sv, 0), lane_f(sv, 16)), fmaxf(lane_f(sv, 32), lane_f(sv, 48)));
        if (lane == 0) s_cm[wave][pr] = sv;
    }
    __syncthreads();
    // the chunk's maximum of each row, for the statistics
    if (t < n_q * G) {
        const int q = t / G, h = h0 + t % G;
        const float m = fmaxf(fmaxf(s_cm[0][t], s_cm[1][t]), fmaxf(s_cm[2][t], s_cm[3][t]));
        S.cmax[((int64_t) (q0 + q) * A.n_head + h) * attn_chunks(A.n_kv) + split] = m;
    }
    // the accumulator the PV launch adds its chunk partials into, zeroed by the launch before it
    if (A.acc) {
        const int nwg = gridDim.x * gridDim.y * gridDim.z;
        const int wg = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
        const int n = A.n_q * A.n_head * HD;
        for (int i = wg * ATT_THREADS + t; i < n; i += nwg * ATT_THREADS) A.acc[i] = 0.0;
    }
}

// one workgroup per (head, query, segment of STATS_SEG positions): the row maximum M from the chunk
// maxima, e = exp(s - M) written over each of the segment's scores (0 throughout a row masked
// everywhere), and the sum of e in double over the segment's positions. The PV launch reads e.
__global__ __launch_bounds__(ATT_THREADS) void attn_stats_kernel(const attn_launch A_) {
    const attn_launch & A = kernargs_prefetched(A_);
    __shared__ float s_m[ATT_WAVES];
    __shared__ double s_s[ATT_WAVES];
    const int h = blockIdx.x, q = blockIdx.y, seg = blockIdx.z;
    const int t = threadIdx.x, lane = t % WAVE, wave = t / WAVE;
    const attn_scratch S = scratch_of(A);
    const int64_t row = (int64_t) q * A.n_head + h;
    float * sc = S.scores + row * A.n_kv;
    const int nch = attn_chunks(A.n_kv);
    // the segment's scores go out first (unused past the end, where a lane loads the element one
    // segment back, or its own first one in the first segment: in bounds, distinct addresses)
    float v[STATS_PER_THREAD];
#pragma unroll
    for (int k = 0; k < STATS_PER_THREAD; k++) {
        const int i = seg * STATS_SEG + k * ATT_THREADS + t;
        v[k] = sc[i < A.n_kv ? i : seg > 0 ? i - STATS_SEG : min(t, A.n_kv - 1)];
    }
    float m = -INFINITY;
    for (int c = t; c < nch; c += ATT_THREADS) m = fmaxf(m, S.cmax[row * nch + c]);
    m = wave_max(m);
    if (lane == 0) s_m[wave] = m;
    __syncthreads();
    float M = s_m[0];
    for (int w = 1; w < ATT_WAVES; w++) M = fmaxf(M, s_m[w]);
    double sum = 0.0;
#pragma unroll
    for (int k = 0; k < STATS_PER_THREAD; k++) {
        const int i = seg * STATS_SEG + k * ATT_THREADS + t;
        const float e = M == -INFINITY ? 0.0f : exp_cr(v[k] - M);
        if (i < A.n_kv) {
            sum += (double) e;
            sc[i] = e;
        }
    }
    sum = wave_sum_d(sum);
    if (lane == 0) s_s[wave] = sum;
    __syncthreads();
    if (t == 0) {
        double tot = 0.0;
        for (int w = 0; w < ATT_WAVES; w++) tot += s_s[w];
        S.ssum[row * attn_segs(A.n_kv) + seg] = tot;
    }
}

// rows (query, head) of one PV workgroup: at most 8 (launch_attn_t picks the queries per workgroup)
constexpr int PV_MAX_ROWS = 8;
constexpr int PV_NP = PV_CHUNK / ATT_WAVES;               // positions per wave
constexpr int PV_SC = (PV_MAX_ROWS * PV_CHUNK + ATT_THREADS - 1) / ATT_THREADS;   // scores per thread
// scores per thread of a PV workgroup that forms its own statistics (FSK below). Measured: 9 (rows
// up to 2304 positions) beats the statistics launch (Llama-3B at 2049: 8.3 us against 6.3 + 4.0);
// 17 (4097 positions, Qwen3-MoE attention) loses (16.5 us against 10.5 + 3.9).
constexpr int PV_FS_SPT = 9;
constexpr int PV_FS_MAX_KV = PV_FS_SPT * ATT_THREADS;

template <int HD>
constexpr int pv_lds_bytes() {
    // [V chunk: PV_CHUNK][HD / 2] dwords, reused for the waves' partials [4][PV_MAX_ROWS][HD] doubles
    return (PV_CHUNK * HD * 2 > ATT_WAVES * PV_MAX_ROWS * HD * 8 ? PV_CHUNK * HD * 2 : ATT_WAVES * PV_MAX_ROWS * HD * 8);
}

// The output of (head h, query q): CMB_PARTS threads per dim each add a consecutive run of the
// chunk partials in chunk order, CMB_PER at a time with all of their loads in flight (a run of
// dependent load -> add would put one round trip per partial on the path), then the runs' sums are
// added in run order (the sums are exact for these operands, so the grouping does not change the
// result); stored as F32 and, with out_q, as Q8_0 blocks.
constexpr int CMB_PARTS = 8;
constexpr int CMB_PER = 9;
template <int HD>
__global__ __launch_bounds__(CMB_PARTS * HD) void attn_combine_kernel(const attn_launch A_, int n_splits) {
    const attn_launch & A = kernargs_prefetched(A_);
    __shared__ double s_run[CMB_PARTS][HD];
    const attn_scratch S = scratch_of(A);
    const int h = blockIdx.x, q = blockIdx.y;
    const int d = threadIdx.x % HD, part = threadIdx.x / HD;
    const double * pp = S.parts + ((int64_t) q * A.n_head + h) * HD + d;
    const int64_t step = (int64_t) A.n_q * A.n_head * HD;
    const int per = (n_splits + CMB_PARTS - 1) / CMB_PARTS;
    const int s0 = part * per, s1 = min(n_splits, s0 + per);
    double acc = 0.0;
    for (int b = s0; b < s1; b += CMB_PER) {
        double v[CMB_PER];
#pragma unroll
        for (int k = 0; k < CMB_PER; k++) v[k] = pp[min(b + k, n_splits - 1) * step];   // clamped, unused past s1
#pragma unroll
        for (int k = 0; k < CMB_PER; k++) acc += b + k < s1 ? v[k] : 0.0;
    }
    s_run[part][d] = acc;
    __syncthreads();
    if (part != 0) return;
    acc = s_run[0][d];
#pragma unroll
    for (int p = 1; p < CMB_PARTS; p++) acc += s_run[p][d];
    const float v = (float) acc;
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

// The combination with the output's Q8_K copy (out_q8k): one workgroup per (256-dim super-block,
// query), CMB_K_PARTS threads per dim adding runs of the chunk partials as above, then the
// super-block quantized with quantize_row_q8_K's arithmetic (the steps of quantize_q8k_kernel: the
// value of largest magnitude, the first on ties; iscale = -127 / max; q = min(127, nearest(iscale *
// x)); d = 1 / iscale; 16-element sums). Every thread reaches every barrier.
constexpr int CMB_K_PARTS = 4;
template <int HD>
__global__ __launch_bounds__(CMB_K_PARTS * 256) void attn_combine_q8k_kernel(const attn_launch A_, int n_splits) {
    const attn_launch & A = kernargs_prefetched(A_);
    __shared__ double s_run[CMB_K_PARTS][256];
    __shared__ float s_ax[4];
    __shared__ int s_idx[4];
    __shared__ float s_val[4];
    __shared__ int s_q[256];
    const attn_scratch S = scratch_of(A);
    const int sb = blockIdx.x, q = blockIdx.y;
    const int t = threadIdx.x, j = t % 256, part = t / 256, lane = t % WAVE, wave = t / WAVE;
    const int h = sb * (256 / HD) + j / HD, d = j % HD;
    const double * pp = S.parts + ((int64_t) q * A.n_head + h) * HD + d;
    const int64_t step = (int64_t) A.n_q * A.n_head * HD;
    const int per = (n_splits + CMB_K_PARTS - 1) / CMB_K_PARTS;
    const int s0 = part * per, s1 = min(n_splits, s0 + per);
    double acc = 0.0;
    for (int b = s0; b < s1; b += CMB_PER) {
        double v[CMB_PER];
#pragma unroll
        for (int k = 0; k < CMB_PER; k++) v[k] = pp[min(b + k, n_splits - 1) * step];   // clamped, unused past s1
#pragma unroll
        for (int k = 0; k < CMB_PER; k++) acc += b + k < s1 ? v[k] : 0.0;
    }
    s_run[part][j] = acc;
    __syncthreads();
    float v = 0.0f;
    if (part == 0) {
        acc = s_run[0][j];
#pragma unroll
        for (int p = 1; p < CMB_K_PARTS; p++) acc += s_run[p][j];
        v = (float) acc;
        A.out[(int64_t) q * A.out_nb1 + (int64_t) h * HD + d] = v;
    }
    // the super-block's value of largest magnitude (waves 0-3 hold its 256 values)
    float ax = fabsf(v);
    int idx = j;
    float val = v;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ax2 = __shfl_xor(ax, o, WAVE);
        const int idx2 = __shfl_xor(idx, o, WAVE);
        const float val2 = __shfl_xor(val, o, WAVE);
        if (ax2 > ax || (ax2 == ax && idx2 < idx)) { ax = ax2; idx = idx2; val = val2; }
    }
    if (part == 0 && lane == 0) { s_ax[wave] = ax; s_idx[wave] = idx; s_val[wave] = val; }
    __syncthreads();
    const int64_t K = (int64_t) A.n_head * HD, nsb = K / 256;
    if (part == 0) {
        float bax = s_ax[0], bval = s_val[0];
        int bidx = s_idx[0];
        for (int w = 1; w < 4; w++) {
            if (s_ax[w] > bax || (s_ax[w] == bax && s_idx[w] < bidx)) { bax = s_ax[w]; bidx = s_idx[w]; bval = s_val[w]; }
        }
        int qv = 0;
        if (bax != 0.0f) {
            const float iscale = -127.f / bval;
            qv = round_half_even(iscale * v);
            qv = qv < 127 ? qv : 127;
            if (j == 0) A.out_q8k.d[q * nsb + sb] = 1 / iscale;
        } else if (j == 0) {
            A.out_q8k.d[q * nsb + sb] = 0.0f;
        }
        A.out_q8k.qs[q * K + (int64_t) sb * 256 + j] = (int8_t) qv;
        s_q[j] = qv;
    }
    __syncthreads();
    if (t < 16) {
        int sum = 0;
        for (int i = 0; i < 16; i++) sum += s_q[t * 16 + i];
        A.out_q8k.bsums[q * (K / 16) + (int64_t) sb * 16 + t] = (int16_t) sum;
    }
}

// FSK > 0 (one query, one head per workgroup, n_kv <= FSK * ATT_THREADS): the workgroup forms its row's
// statistics itself, from the chunk maxima and every score of the row, instead of reading them from
// the statistics launch; the sum is the statistics kernel's, exp(s - M) in double over the row's
// positions (exact in practice, so its grouping does not matter), and e = exp(s - M) of the chunk's
// positions is formed here too. The statistics launch is not made.
template <int HD, int G, int FSK>
__global__ __launch_bounds__(ATT_THREADS) void attn_pv_kernel(const attn_launch A_, int pvq) {
    const attn_launch & A = kernargs_prefetched(A_);
    constexpr int HD2 = HD / 2;
    constexpr int PIECES = HD / 8;                        // 16-byte pieces per V row
    constexpr int ITER = PV_CHUNK * PIECES / ATT_THREADS;
    __shared__ __align__(16) uint8_t s_buf[pv_lds_bytes<HD>()];
    __shared__ __align__(16) double s_p[PV_MAX_ROWS][PV_CHUNK];
    __shared__ float s_M[PV_MAX_ROWS], s_inv[PV_MAX_ROWS];
    uint32_t * s_v = (uint32_t *) s_buf;                  // [PV_CHUNK][HD2]
    double * s_part = (double *) s_buf;                   // [ATT_WAVES][PV_MAX_ROWS][HD], after the dots
    const int split = blockIdx.x, h0 = blockIdx.y * G;   // as in the scores kernel
    const int kvh = __builtin_amdgcn_readfirstlane(div_small(h0, A.s_inv_gqa));
    const int t = threadIdx.x, lane = t % WAVE, wave = t / WAVE;
    const int t0 = split * PV_CHUNK;
    const int nt = min(PV_CHUNK, A.n_kv - t0);
    const int q0 = blockIdx.z * pvq;                  // this workgroup's queries: q0 .. q0 + pvq - 1
    const int n_rows = min(pvq, A.n_q - q0) * G;      // <= PV_MAX_ROWS (pvq = PV_MAX_ROWS / G or 1)
    const attn_scratch S = scratch_of(A);
    const int nseg = attn_segs(A.n_kv);
    // scratch row of workgroup row pr (32-bit: launch_attn_decode checks the scratch indices)
    auto row_of = [&](int pr) { return (q0 + pr / G) * A.n_head + h0 + pr % G; };

    // loads, in the order they are needed (they complete in issue order): the chunk's scores of
    // every row (with the statistics launch: its e values), the segment sums, then the chunk's V
    // rows (16-byte pieces). Indices clamped, values past the ends unused.
    float sc[PV_SC];
#pragma unroll
    for (int k = 0; k < PV_SC; k++) {
        const int i = wrap_index(t + k * ATT_THREADS, n_rows * PV_CHUNK, t);
        const int pr = i / PV_CHUNK, tt = tail_row(i % PV_CHUNK, nt, t0, PV_CHUNK);
        sc[k] = S.scores[row_of(pr) * A.n_kv + t0 + tt];
    }
    float rmax = 0.0f;
    double ssum = 0.0, seg_sum = 0.0;
    constexpr bool FS = FSK > 0;
    constexpr int FR = FS ? G : 1, FK = FS ? FSK : 1;
    float cm[FR], fv[FR][FK];
    if constexpr (FS) {
        // each row's chunk maxima (nch <= ATT_THREADS) and scores (FSK per thread)
        const int nch = attn_chunks(A.n_kv);
#pragma unroll
        for (int r = 0; r < G; r++) cm[r] = S.cmax[row_of(r) * nch + min(t, nch - 1)];
#pragma unroll
        for (int r = 0; r < G; r++) {
#pragma unroll
            for (int k = 0; k < FK; k++) fv[r][k] = S.scores[row_of(r) * A.n_kv + wrap_index(t + k * ATT_THREADS, A.n_kv, t)];
        }
    } else if (n_rows * nseg <= ATT_THREADS) {
        // one segment sum per thread, issued with the other loads (a loop of dependent loads here
        // would hold back the V loads below); added per row after the loads
        if (t < n_rows * nseg) seg_sum = S.ssum[row_of(t / nseg) * nseg + t % nseg];
    } else if (t < n_rows) {
        for (int k = 0; k < nseg; k++) ssum += S.ssum[row_of(t) * nseg + k];   // segment order
    }
    uint4 vv[ITER];
    const __half * vbase = A.v + kvh * A.v_nb1 + t0 * A.v_nb2;
#pragma unroll
    for (int it = 0; it < ITER; it++) {
        const unsigned pc = t + it * ATT_THREADS;
        const unsigned r = pc / PIECES, c = pc % PIECES;
        vv[it] = *(const uint4 *) (vbase + (tail_row((int) r, nt, t0, PV_CHUNK) * A.v_s2 + (int) c * 8));
    }
    // rows staged as zero: padding rows past the end (their loads read the last row; no term) and,
    // with skip_masked, rows masked for every query of the workgroup (their p is 0 for every row).
    // Applied when the rows are stored to LDS: zeroing a register right after its load would make
    // the compiler wait for every load issued so far.
    bool vzero[ITER];
#pragma unroll
    for (int it = 0; it < ITER; it++) vzero[it] = (t + it * ATT_THREADS) / PIECES >= nt;
    if (A.skip_masked && A.mask) {
        const int nq = min(pvq, A.n_q - q0);
#pragma unroll
        for (int it = 0; it < ITER; it++) {
            const int r = (t + it * ATT_THREADS) / PIECES;
            bool dead = r < nt;
            for (int q = 0; q < nq && dead; q++) dead = mask_at(A, q0 + q, t0 + r) == -INFINITY;
            vzero[it] = vzero[it] || dead;
        }
    }
    if constexpr (FS) {
        __shared__ float s_fm[ATT_WAVES][FR];
        __shared__ double s_fs[ATT_WAVES][FR];
#pragma unroll
        for (int r = 0; r < G; r++) {
            const float m = wave_max(cm[r]);
            if (lane == 0) s_fm[wave][r] = m;
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < G; r++) {
            const float M = fmaxf(fmaxf(s_fm[0][r], s_fm[1][r]), fmaxf(s_fm[2][r], s_fm[3][r]));
            // every exp evaluated (clamped positions repeat a valid score) and the ones past the
            // end dropped, so that the independent evaluations interleave
            double a = 0.0;
            if (M != -INFINITY) {
                double e[FK];
#pragma unroll
                for (int k = 0; k < FK; k++) e[k] = (double) exp_cr(fv[r][k] - M);
#pragma unroll
                for (int k = 0; k < FK; k++) a += t + k * ATT_THREADS < A.n_kv ? e[k] : 0.0;
            }
            a = wave_sum_d(a);
            if (lane == 0) s_fs[wave][r] = a;
        }
        __syncthreads();
        if (t < G) {
            rmax = fmaxf(fmaxf(s_fm[0][t], s_fm[1][t]), fmaxf(s_fm[2][t], s_fm[3][t]));
            ssum = ((s_fs[0][t] + s_fs[1][t]) + s_fs[2][t]) + s_fs[3][t];
        }
    }
    if (!FS && n_rows * nseg <= ATT_THREADS) {
        double * s_seg = &s_p[0][0];  // s_p is not yet in use: the segment sums, [row][segment]
        s_seg[t] = seg_sum;
        __syncthreads();
        if (t < n_rows) {
            for (int k = 0; k < nseg; k++) ssum += s_seg[t * nseg + k];   // segment order
        }
        __syncthreads();
    }
    if (t < n_rows) {
        s_M[t] = rmax;
        s_inv[t] = ssum > 0.0 ? (float) (1.0 / ssum) : 0.0f;
    }
    __syncthreads();
    // p = F16(e * (1/S)) for the chunk's positions, e = exp(s - M) (formed here with FSK, read from
    // the statistics launch otherwise); 0 past the end; with p_f32 not rounded to F16; kept as
    // doubles
#pragma unroll
    for (int k = 0; k < PV_SC; k++) {
        const int i = t + k * ATT_THREADS;
        if (i < n_rows * PV_CHUNK) {
            const int pr = i / PV_CHUNK, tt = i % PV_CHUNK;
            float p = 0.0f;
            if (tt < nt) {
                float e = sc[k];
                if constexpr (FS) {
                    const float M = s_M[pr];
                    e = M == -INFINITY ? 0.0f : exp_cr(sc[k] - M);
                }
                p = as_f32(e * s_inv[pr]);
                if (!A.p_f32) p = __half2float(__float2half_rn(p));
            }
            s_p[pr][tt] = (double) p;
        }
    }
#pragma unroll
    for (int it = 0; it < ITER; it++) {
        const int pc = t + it * ATT_THREADS;
        const int r = pc / PIECES, c = pc % PIECES;
        uint32_t * d = s_v + r * HD2 + c * 4;
        const bool z = vzero[it];
        d[0] = z ? 0u : vv[it].x; d[1] = z ? 0u : vv[it].y; d[2] = z ? 0u : vv[it].z; d[3] = z ? 0u : vv[it].w;
    }
    __syncthreads();

    // P V over this wave's positions (lane: dims 2 lane, 2 lane + 1): each V value widened once and
    // multiplied into up to four rows at a time; a product of two F16 values is exact in double, so
    // fma(p, v, acc) rounds as acc + p*v does (the sums are exact for these operands)
    const int d2 = min(lane, HD2 - 1);
    // rows r0 .. r0 + NR - 1 (clamped; rows past n_rows are computed and dropped): NR = 4, or the
    // G rows of a launch that forms its own statistics (one query), all of which are live
    constexpr int NR = FS ? G : 4;
    static_assert(NR <= 4, "PV rows per pass");
    auto dot_rows = [&](int r0, double (&acc)[4][2]) {
#pragma unroll
        for (int r = 0; r < 4; r++) acc[r][0] = acc[r][1] = 0.0;
#pragma unroll 4
        for (int j = 0; j < PV_NP; j++) {
            const int tt = wave * PV_NP + j;
            const float2 vf = __half22float2(*(const __half2 *) &s_v[tt * HD2 + d2]);
            const double v0 = (double) vf.x, v1 = (double) vf.y;
#pragma unroll
            for (int r = 0; r < NR; r++) {
                const double p = s_p[min(r0 + r, PV_MAX_ROWS - 1)][tt];
                acc[r][0] = fma(p, v0, acc[r][0]);
                acc[r][1] = fma(p, v1, acc[r][1]);
            }
        }
    };
    double acc_a[4][2], acc_b[4][2];
    dot_rows(0, acc_a);
    if (n_rows > 4) dot_rows(4, acc_b);
    __syncthreads();                                  // every wave is done with the V chunk
    if (lane < HD2) {
#pragma unroll
        for (int r = 0; r < PV_MAX_ROWS; r++) {
            if (r < n_rows) {
                const double a0 = r < 4 ? acc_a[r % 4][0] : acc_b[r % 4][0];
                const double a1 = r < 4 ? acc_a[r % 4][1] : acc_b[r % 4][1];
                s_part[(wave * PV_MAX_ROWS + r) * HD + 2 * lane] = a0;
                s_part[(wave * PV_MAX_ROWS + r) * HD + 2 * lane + 1] = a1;
            }
        }
    }
    __syncthreads();
    // the chunk's partial of each (row, dim): the waves' sums added in wave order
    for (int i = t; i < n_rows * HD; i += ATT_THREADS) {
        const int r = i / HD, d = i % HD;
        const double v = ((s_part[(0 * PV_MAX_ROWS + r) * HD + d] + s_part[(1 * PV_MAX_ROWS + r) * HD + d]) +
                          s_part[(2 * PV_MAX_ROWS + r) * HD + d]) + s_part[(3 * PV_MAX_ROWS + r) * HD + d];
        const int q = q0 + r / G, h = h0 + r % G;
        if (A.acc) unsafeAtomicAdd(A.acc + ((int64_t) q * A.n_head + h) * HD + d, v);
        else S.parts[(((int64_t) split * A.n_q + q) * A.n_head + h) * HD + d] = v;
    }
}

// ---------------------------------------------------------------------------------------------
// Multi-query decode (more than ATT_MAX_Q queries, RoPE not folded in): the scores and PV launches
// on the f64 matrix cores, with the statistics and combine launches above unchanged. The rows of a
// KV head are its (query, head) pairs, row r = q * G + (h - kvh * G) for the G heads of the KV
// head, in tiles of 16 (one MFMA row tile per workgroup). Same sums as the chain: the F16 x F16
// products are exact in double and their double sums exact for these operands in practice, so the
// matrix cores' accumulation order gives the same floats as the kernels above.
// f64 MFMA 16x16x4 lane layout: A[i][k] at lane i + 16k, B[k][j] at lane j + 16k, D[i][j] in
// register i / 4 of lane j + 16 (i % 4).
typedef double v4d __attribute__((ext_vector_type(4)));

constexpr int MQ_ROWS = 16;


__host__ __device__ inline int mq_tiles(const attn_launch & A) {
    return (A.n_q * (A.n_head / A.n_head_kv) + MQ_ROWS - 1) / MQ_ROWS;
}

// (64-position chunk, KV head, row tile) workgroups; wave w takes positions 16 w .. 16 w + 15 of the
// chunk. Writes the scores (kq * scale + mask) and each row's chunk maximum, as attn_scores_kernel.
template <int HD>
__global__ __launch_bounds__(ATT_THREADS) void attn_scores_mq_kernel(const attn_launch A_) {
    const attn_launch & A = kernargs_prefetched(A_);
    constexpr int KSTR = HD + 2;                  // halves per staged K row (one dword of padding)
    constexpr int PIECES = HD / 8;                // 16-byte pieces per K row
    constexpr int ITER = ATT_CHUNK * PIECES / ATT_THREADS;
    static_assert(ATT_CHUNK * PIECES % ATT_THREADS == 0, "whole 16-byte pieces per thread");
    constexpr int NJ = HD / 4;                    // 4-dim MFMA steps
    static_assert(NJ % 2 == 0, "pairs of 4-dim steps");
    // Q tile rows of QSTR floats: the 16 rows x 4 dims that one MFMA operand read takes fall on 64
    // distinct banks
    constexpr int QSTR = HD + 4;
    constexpr int QPT = HD / 16;                  // Q elements per thread: 16 threads per tile row
    static_assert(MQ_ROWS * 16 == ATT_THREADS && QPT % 2 == 0, "one tile row per 16 threads");
    __shared__ __align__(16) __half s_k[ATT_CHUNK * KSTR];
    __shared__ __align__(16) float s_q[MQ_ROWS * QSTR];
    __shared__ float s_cm[ATT_WAVES][MQ_ROWS];
    const int split = blockIdx.x, kvh = blockIdx.y, r0 = blockIdx.z * MQ_ROWS;
    const int G = A.n_head / A.n_head_kv, n_rows = A.n_q * G;
    const float inv_g = 1.0f / (float) G;
    const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
    const int t0 = split * ATT_CHUNK, nt = min(ATT_CHUNK, A.n_kv - t0);
    const attn_scratch S = scratch_of(A);

    // Loads first, all unconditional at clamped indices (32-bit offsets: the launch checks that
    // every index fits): the tile's Q rows once per workgroup, QPT consecutive dims per thread (rows
    // past n_rows repeat the last row, their results are not stored); the mask of the lane's four
    // outputs (rows g + 4 r, g = lane / 16, at position 16 wave + lane % 16; an F32 and an F16 load,
    // the one of the other type reading Q); then the chunk's K rows.
    const int qi = threadIdx.x / 16, qd0 = (threadIdx.x % 16) * QPT;
    float qf[QPT];
    {
        const int ra = min(r0 + qi, n_rows - 1), qa = div_small(ra, inv_g);
        const float * src = A.q + ((kvh * G + ra - qa * G) * (int) A.q_nb1 + qa * (int) A.q_nb2 + qd0);
#pragma unroll
        for (int k = 0; k < QPT; k++) qf[k] = src[k];
    }
    const int tl = wave * 16 + lane % 16;          // the lane's position in the chunk
    const int tc = t0 + min(tl, nt - 1);
    const bool mask32 = A.mask && !A.mask_f16, mask16 = A.mask && A.mask_f16;
    const int mstride = (int) (A.mask_nb1 >> (A.mask_f16 ? 1 : 2));   // elements per mask row
    const float * mrow32 = (const float *) (mask32 ? A.mask : (const void *) A.q);
    const __half * mrow16 = (const __half *) (mask16 ? A.mask : (const void *) A.q);
    float m32[4];
    __half m16[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int mi = div_small(min(r0 + lane / 16 + 4 * r, n_rows - 1), inv_g) * mstride + tc;
        m32[r] = mrow32[mask32 ? mi : 0];
        m16[r] = mrow16[mask16 ? mi : 0];
    }
    uint4 kv[ITER];
    {
        const __half * kbase = A.k + kvh * A.k_nb1;
        const int kst = (int) A.k_nb2;
#pragma unroll
        for (int it = 0; it < ITER; it++) {
            const int pc = threadIdx.x + it * ATT_THREADS;
            const int r = pc / PIECES, c = pc % PIECES;
            kv[it] = *(const uint4 *) (kbase + ((t0 + tail_row(r, nt, t0, ATT_CHUNK)) * kst + c * 8));
        }
    }
    __builtin_amdgcn_sched_barrier(0);            // every load above is out before any wait
    // Q rounded to F16 (the mul_mat's conversion of its F32 operand)
#pragma unroll
    for (int k = 0; k < QPT; k += 2) {
        *(float2 *) (s_q + qi * QSTR + qd0 + k) =
            make_float2(__half2float(__float2half_rn(qf[k])), __half2float(__float2half_rn(qf[k + 1])));
    }
    float mk[4];
#pragma unroll
    for (int r = 0; r < 4; r++) mk[r] = mask32 ? m32[r] : mask16 ? __half2float(m16[r]) : 0.0f;
    // K rows to LDS, zero past nt (their loads read the last row)
#pragma unroll
    for (int it = 0; it < ITER; it++) {
        const int pc = threadIdx.x + it * ATT_THREADS;
        const int r = pc / PIECES, c = pc % PIECES;
        uint32_t * d = (uint32_t *) (s_k + r * KSTR + c * 8);
        const bool z = r >= nt;
        d[0] = z ? 0u : kv[it].x; d[1] = z ? 0u : kv[it].y; d[2] = z ? 0u : kv[it].z; d[3] = z ? 0u : kv[it].w;
    }
    __syncthreads();

    // S[row][position] over the head dims, two accumulation chains (added at the end; the double
    // sums are exact for these operands, so the grouping does not matter)
    // (A operand: lane (i + 16 k) holds Q[row i][4 j + k]; B: lane (j + 16 k) holds K[position j][4 j' + k])
    v4d acc = { 0.0, 0.0, 0.0, 0.0 }, acc2 = { 0.0, 0.0, 0.0, 0.0 };
    const __half * kr = s_k + tl * KSTR + lane / 16;
    const float * qr = s_q + (lane % 16) * QSTR + lane / 16;
#pragma unroll
    for (int j = 0; j < NJ; j += 2) {
        const double a = (double) qr[4 * j], a2 = (double) qr[4 * j + 4];
        const double b = (double) __half2float(kr[4 * j]), b2 = (double) __half2float(kr[4 * j + 4]);
        acc = __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, acc, 0, 0, 0);
        acc2 = __builtin_amdgcn_mfma_f64_16x16x4f64(a2, b2, acc2, 0, 0, 0);
    }
    acc += acc2;
    // the softmax input as the graph forms it, (float) kq * scale + mask (-inf where masked, without
    // the dot); -inf past the chunk's end (not stored, no part in the maximum)
    float sv[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int rr = r0 + lane / 16 + 4 * r;
        sv[r] = tl >= nt ? -INFINITY : mk[r] == -INFINITY ? -INFINITY : (float) acc[r] * A.scale + mk[r];
        if (tl < nt && rr < n_rows) {
            const int qq = div_small(rr, inv_g);
            S.scores[(qq * A.n_head + kvh * G + rr - qq * G) * A.n_kv + t0 + tl] = sv[r];
        }
    }
    // each row's maximum over the wave's 16 positions (the 16 lanes of one DPP row), then over the
    // four waves
#pragma unroll
    for (int r = 0; r < 4; r++) {
        float m = sv[r];
        m = fmaxf(m, dpp_f<0xB1>(m));
        m = fmaxf(m, dpp_f<0x4E>(m));
        m = fmaxf(m, dpp_f<0x141>(m));
        m = fmaxf(m, dpp_f<0x140>(m));
        if (lane % 16 == 0) s_cm[wave][lane / 16 + 4 * r] = m;
    }
    __syncthreads();
    if (threadIdx.x < MQ_ROWS && r0 + (int) threadIdx.x < n_rows) {
        const int rr = r0 + threadIdx.x, i = threadIdx.x, qq = div_small(rr, inv_g);
        const int row = qq * A.n_head + kvh * G + rr - qq * G;
        S.cmax[row * attn_chunks(A.n_kv) + split] = fmaxf(fmaxf(s_cm[0][i], s_cm[1][i]), fmaxf(s_cm[2][i], s_cm[3][i]));
    }
}

// (128-position chunk, KV head, row tile) workgroups: p = F16(e * (1/S)) of the tile's rows over the
// chunk (e = exp(s - M) from the statistics launch; P32: p kept a float, flash_attn_ext), then the
// chunk's partial P V of every (row, dim); wave w takes the 16-dim output tiles w, w + 4, ... over
// all of the chunk's positions, so no partials are added across waves.
template <int HD, bool P32>
__global__ __launch_bounds__(ATT_THREADS) void attn_pv_mq_kernel(const attn_launch A_) {
    const attn_launch & A = kernargs_prefetched(A_);
    constexpr int PIECES = HD / 8;                // 16-byte pieces per V row
    constexpr int ITER = PV_CHUNK * PIECES / ATT_THREADS;
    static_assert(PV_CHUNK * PIECES % ATT_THREADS == 0, "whole 16-byte pieces per thread");
    constexpr int NT = HD / 16;                   // 16-dim output tiles
    constexpr int TPW = (NT + ATT_WAVES - 1) / ATT_WAVES;
    constexpr int NS = PV_CHUNK / 4;              // 4-position MFMA steps
    constexpr int EPT = PV_CHUNK / 16;            // positions per thread: 16 threads per tile row
    static_assert(MQ_ROWS * 16 == ATT_THREADS && EPT == 8, "one tile row per 16 threads, 8 positions each");
    // p rows: the 16 rows x 4 positions of one A operand read fall on distinct banks (F16: pairs
    // of lanes share a dword)
    using pt = typename std::conditional<P32, float, __half>::type;
    constexpr int PSTR = P32 ? PV_CHUNK + 4 : PV_CHUNK + 8;
    // V in the order the MFMA B operand reads it: step s, tile, lane j + 16 k -> V[4 s + k][16 tile + j]
    __shared__ __align__(16) __half s_v[PV_CHUNK * HD];
    __shared__ __align__(16) pt s_p[MQ_ROWS * PSTR];
    const int split = blockIdx.x, kvh = blockIdx.y, r0 = blockIdx.z * MQ_ROWS;
    const int G = A.n_head / A.n_head_kv, n_rows = A.n_q * G;
    const int t = threadIdx.x, lane = t % WAVE, wave = t / WAVE;
    const int t0 = split * PV_CHUNK, nt = min(PV_CHUNK, A.n_kv - t0);
    const attn_scratch S = scratch_of(A);
    const int nseg = attn_segs(A.n_kv);
    // this thread's tile row and positions: row pr, positions pp0 .. pp0 + 7 of the chunk
    const int pr = t / 16, pp0 = (t % 16) * EPT;
    const float inv_g = 1.0f / (float) G;
    const int rr = min(r0 + pr, n_rows - 1);      // clamped: rows past n_rows are not stored
    const int rq = div_small(rr, inv_g);
    const int row = rq * A.n_head + kvh * G + rr - rq * G;

    // loads, in the order they are needed (they complete in issue order): the e values of the
    // thread's positions, its row's segment sums (one per thread of the row while they fit), then
    // the chunk's V rows. Indices clamped (32-bit offsets: the launch checks that every index
    // fits), values past the ends unused.
    float ev[EPT];
    {
        const float * esrc = S.scores + (row * A.n_kv + t0);
#pragma unroll
        for (int k = 0; k < EPT; k++) ev[k] = esrc[tail_row(pp0 + k, nt, t0, PV_CHUNK)];
    }
    const bool seg_lanes = nseg <= 16;
    const double seg_sum = S.ssum[row * nseg + min(t % 16, nseg - 1)];
    uint4 vv[ITER];
    {
        const __half * vbase = A.v + kvh * A.v_nb1;
        const int vst = (int) A.v_nb2;
#pragma unroll
        for (int it = 0; it < ITER; it++) {
            const int pc = t + it * ATT_THREADS;
            const int r = pc / PIECES, c = pc % PIECES;
            vv[it] = *(const uint4 *) (vbase + ((t0 + tail_row(r, nt, t0, PV_CHUNK)) * vst + c * 8));
        }
    }
    // V rows staged as zero: padding rows past the end and, with skip_masked, rows masked for every
    // query of the tile (p is 0 there for every row, and 0 * a non-finite V must not reach the sums).
    // Applied at the LDS store: zeroing a register right after its load makes the compiler wait for
    // every load issued so far.
    bool vzero[ITER];
#pragma unroll
    for (int it = 0; it < ITER; it++) vzero[it] = (t + it * ATT_THREADS) / PIECES >= nt;
    if (A.skip_masked && A.mask) {
        const int qa = div_small(r0, inv_g), qb = div_small(min(r0 + MQ_ROWS, n_rows) - 1, inv_g);
#pragma unroll
        for (int it = 0; it < ITER; it++) {
            const int r = (t + it * ATT_THREADS) / PIECES;
            bool dead = r < nt;
            for (int q = qa; q <= qb && dead; q++) dead = mask_at(A, q, t0 + r) == -INFINITY;
            vzero[it] = vzero[it] || dead;
        }
    }
    // the row's S: its segment sums added in segment order (read from the row's 16 lanes, or
    // loaded one after another past 16 segments)
    double ssum = 0.0;
    if (seg_lanes) {
        for (int k = 0; k < nseg; k++) ssum += __shfl(seg_sum, (lane & ~15) + k, WAVE);
    } else {
        for (int k = 0; k < nseg; k++) ssum += S.ssum[row * nseg + k];
    }
    const float inv = ssum > 0.0 ? (float) (1.0 / ssum) : 0.0f;
    // p (0 past the end; rounded to F16 unless P32), eight consecutive positions per store
    {
        pt pv8[EPT];
#pragma unroll
        for (int k = 0; k < EPT; k++) {
            // formed for every position (past the end from a repeated e) and selected after, so
            // that no lane branches
            const float p = as_f32(ev[k] * inv);
            if constexpr (P32) pv8[k] = pp0 + k < nt ? p : 0.0f;
            else pv8[k] = pp0 + k < nt ? __float2half_rn(p) : __float2half_rn(0.0f);
        }
        uint4 w[EPT * sizeof(pt) / 16];
        __builtin_memcpy(w, pv8, sizeof(w));
        uint4 * d = (uint4 *) (s_p + pr * PSTR + pp0);
#pragma unroll
        for (int k = 0; k < (int) (EPT * sizeof(pt) / 16); k++) d[k] = w[k];
    }
    // V pieces: row r = 4 s + k, dims 8 c .. 8 c + 7 = tile c / 2, j = 8 (c % 2) .. + 7
#pragma unroll
    for (int it = 0; it < ITER; it++) {
        const int pc = t + it * ATT_THREADS;
        const int r = pc / PIECES, c = pc % PIECES;
        const bool z = vzero[it];
        *(uint4 *) (s_v + (((r / 4) * NT + c / 2) * 4 + r % 4) * 16 + 8 * (c % 2)) =
            z ? make_uint4(0u, 0u, 0u, 0u) : vv[it];
    }
    __syncthreads();

    // out[row][16 tile + j] += sum over the chunk's positions of p[row][pos] V[pos][16 tile + j]; one
    // accumulation chain per output tile (A operand: lane (i + 16 k) holds p[row i][4 s + k])
    v4d acc[TPW];
#pragma unroll
    for (int k = 0; k < TPW; k++) acc[k] = v4d{ 0.0, 0.0, 0.0, 0.0 };
    const pt * pa = s_p + (lane % 16) * PSTR + lane / 16;
#pragma unroll 4
    for (int s = 0; s < NS; s++) {
        const double a = (double) (float) pa[4 * s];
#pragma unroll
        for (int k = 0; k < TPW; k++) {
            const int tile = wave + ATT_WAVES * k;
            if (tile < NT) {
                const double b = (double) __half2float(s_v[(s * NT + tile) * WAVE + lane]);
                acc[k] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, acc[k], 0, 0, 0);
            }
        }
    }
    // register r of lane (c + 16 g): row g + 4 r, dim 16 tile + c
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int ro = r0 + lane / 16 + 4 * r;
        if (ro >= n_rows) continue;
        const int q = div_small(ro, inv_g), h = kvh * G + ro - q * G;
        double * dst = S.parts + (((split * A.n_q + q) * A.n_head + h) * HD + lane % 16);
#pragma unroll
        for (int k = 0; k < TPW; k++) {
            const int tile = wave + ATT_WAVES * k;
            if (tile < NT) dst[16 * tile] = acc[k][r];
        }
    }
}

// the combination launch: with out_q8k the Q8_K variant (one workgroup per 256-dim super-block)
template <int HD>
static void launch_combine(const attn_launch & A, int pv_splits, hipStream_t st) {
    if constexpr (256 % HD == 0) {
        if (A.out_q8k.qs) {
            return launch(attn_combine_q8k_kernel<HD>, dim3(A.n_head * HD / 256, A.n_q), dim3(CMB_K_PARTS * 256), 0, st, A,
                          pv_splits);
        }
    }
    if (A.out_q8k.qs) HIP_ABORT("attn: a Q8_K output needs 256 %% hd == 0");
    launch(attn_combine_kernel<HD>, dim3(A.n_head, A.n_q), dim3(CMB_PARTS * HD), 0, st, A, pv_splits);
}

template <int HD>
static void launch_attn_mq(const attn_launch & A, hipStream_t st) {
    const int splits = attn_chunks(A.n_kv);
    const int pv_splits = (A.n_kv + PV_CHUNK - 1) / PV_CHUNK;
    const int tiles = mq_tiles(A);
    // the kernels' quotient by the GQA group and their 32-bit offsets
    const int64_t G = A.n_head / A.n_head_kv, lim = INT32_MAX;
    if (A.n_q * G >= DIV_SMALL_MAX || G > 64) HIP_ABORT("attn: %d queries x %d heads per KV head past the multi-query rows", A.n_q, (int) G);
    const bool fits = (A.n_head - 1) * A.q_nb1 + (A.n_q - 1) * A.q_nb2 + HD <= lim &&
                      (A.n_head_kv - 1) * A.k_nb1 + (int64_t) (A.n_kv - 1) * A.k_nb2 + HD <= lim &&
                      (A.n_head_kv - 1) * A.v_nb1 + (int64_t) (A.n_kv - 1) * A.v_nb2 + HD <= lim &&
                      (!A.mask || (A.n_q - 1) * (A.mask_nb1 / (A.mask_f16 ? 2 : 4)) + A.n_kv <= lim) &&
                      (int64_t) A.n_q * A.n_head * A.n_kv <= lim && (int64_t) pv_splits * A.n_q * A.n_head * HD <= lim;
    if (!fits) HIP_ABORT("attn: multi-query operands past 32-bit element offsets");
    launch(attn_scores_mq_kernel<HD>, dim3(splits, A.n_head_kv, tiles), dim3(ATT_THREADS), 0, st, A);
    launch(attn_stats_kernel, dim3(A.n_head, A.n_q, attn_segs(A.n_kv)), dim3(ATT_THREADS), 0, st, A);
    if (A.p_f32) launch((attn_pv_mq_kernel<HD, true>), dim3(pv_splits, A.n_head_kv, tiles), dim3(ATT_THREADS), 0, st, A);
    else launch((attn_pv_mq_kernel<HD, false>), dim3(pv_splits, A.n_head_kv, tiles), dim3(ATT_THREADS), 0, st, A);
    launch_combine<HD>(A, pv_splits, st);
}

template <int HD, int G>
static void launch_attn_t(const attn_launch & A, hipStream_t st) {
    const int splits = (A.n_kv + ATT_CHUNK - 1) / ATT_CHUNK;
    const int pv_splits = (A.n_kv + PV_CHUNK - 1) / PV_CHUNK;
    const int qz = (A.n_q + ATT_MAX_Q - 1) / ATT_MAX_Q;   // groups of up to ATT_MAX_Q queries
    // G: heads per workgroup (the GQA group, or a part of it); grid.y = head groups
    const size_t dyn = scores_dyn_floats<HD, G>(std::min(A.n_q, ATT_MAX_Q)) * sizeof(float);
    static bool big_lds = false;
    if (dyn > 32768 && !big_lds) {
        HIP_CHECK(hipFuncSetAttribute((const void *) attn_scores_kernel<HD, G>, hipFuncAttributeMaxDynamicSharedMemorySize, 98304));
        big_lds = true;
    }
    launch((attn_scores_kernel<HD, G>), dim3(splits, A.n_head / G, qz), dim3(ATT_THREADS), dyn, st, A);
    static_assert(G <= PV_MAX_ROWS, "PV rows");
    const int pvq = std::max(1, std::min(ATT_MAX_Q, PV_MAX_ROWS / G));   // queries per PV workgroup
    const dim3 pv_grid(pv_splits, A.n_head / G, (A.n_q + pvq - 1) / pvq);
    if (A.n_q == 1 && A.n_kv <= PV_FS_MAX_KV) {
        // one head per workgroup: each workgroup evaluates the exp of every score of its rows
        launch((attn_pv_kernel<HD, 1, PV_FS_SPT>), dim3(pv_splits, A.n_head, 1), dim3(ATT_THREADS), 0, st, A, 1);
    } else {
        launch(attn_stats_kernel, dim3(A.n_head, A.n_q, attn_segs(A.n_kv)), dim3(ATT_THREADS), 0, st, A);
        launch((attn_pv_kernel<HD, G, 0>), pv_grid, dim3(ATT_THREADS), 0, st, A, pvq);
    }
    if (!A.acc) launch_combine<HD>(A, pv_splits, st);
}

template <int HD>
static void launch_attn_hd(const attn_launch & A, hipStream_t st) {
    // heads per workgroup: the GQA group, halved while a workgroup would hold more than 4 (query,
    // head) rows for one query, 8 for several (more workgroups with fewer rows each; the split
    // workgroups of a KV head read its K and V chunk each, mostly from L2). Measured: one query
    // with 8 heads per KV head runs best at 4 heads per workgroup, 16-query steps at 2.
    const int G = A.n_head / A.n_head_kv;
    const int max_rows = A.n_q > 1 ? 8 : 4;
    int hp = G;
    while (hp % 2 == 0 && hp * std::min(A.n_q, ATT_MAX_Q) > max_rows) hp /= 2;
    switch (hp) {
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

// The decode kernels' source rows with 32-bit element strides (attn_launch::sq and the fields after
// it), checked so that every per-lane offset the kernels form fits 32 bits.
static attn_launch resolve_sources(const attn_launch & A) {
    attn_launch B = A;
    const bool qnorm = A.rope && A.qn.x, knorm = A.rope && A.kn.x;
    int64_t q1 = A.q_nb1, q2 = A.q_nb2;
    B.sq = A.q;
    if (A.rope) {
        B.sq = qnorm ? A.qn.x : (const float *) A.rq.src.data;
        q1 = qnorm ? A.qn.nb1 : A.rq.src.nb[1] / 4;
        q2 = qnorm ? A.qn.nb2 : A.rq.src.nb[2] / 4;
    }
    int64_t k1 = q1, k2 = q2, v1 = q1, v2 = q2;
    B.sk = B.sv = B.sq;
    if (A.rope) {
        B.sk = knorm ? A.kn.x : (const float *) A.rk.src.data;
        k1 = knorm ? A.kn.nb1 : A.rk.src.nb[1] / 4;
        k2 = knorm ? A.kn.nb2 : A.rk.src.nb[2] / 4;
        B.sv = (const float *) A.rv.src.data;
        v1 = A.rv.src.nb[1] / 4;
        v2 = A.rv.src.nb[2] / 4;
    }
    B.sqw = qnorm ? A.qn.w : B.sq;
    B.skw = knorm ? A.kn.w : B.sq;
    B.spos = A.rope ? A.rq.pos : (const int32_t *) B.sq;
    B.s_half = A.rope ? A.rq.p.n_dims / 2 : 1;
    const int64_t ms = A.mask ? A.mask_nb1 / (A.mask_f16 ? 2 : 4) : 0;
    const int64_t lim = INT32_MAX;
    const bool fits = (A.n_head - 1) * q1 + (A.n_q - 1) * q2 + A.hd <= lim &&
                      (A.n_head_kv - 1) * k1 + (A.n_q - 1) * k2 + A.hd <= lim &&
                      (A.n_head_kv - 1) * v1 + (A.n_q - 1) * v2 + A.hd <= lim &&
                      std::max(ATT_CHUNK, PV_CHUNK) * std::max(A.k_nb2, A.v_nb2) + A.hd <= lim &&
                      (A.n_q - 1) * ms + A.n_kv <= lim && q1 >= 0 && q2 >= 0 && k1 >= 0 && k2 >= 0 && v1 >= 0 && v2 >= 0 &&
                      (int64_t) A.n_q * A.n_head * A.n_kv <= lim &&
                      (int64_t) (A.n_kv + PV_CHUNK - 1) / PV_CHUNK * A.n_q * A.n_head * A.hd <= lim;
    if (!fits) HIP_ABORT("attn: operand strides past 32-bit element offsets");
    B.sq1 = (int32_t) q1; B.sq2 = (int32_t) q2;
    B.sk1 = (int32_t) k1; B.sk2 = (int32_t) k2;
    B.sv1 = (int32_t) v1; B.sv2 = (int32_t) v2;
    B.s_mask_stride = (int32_t) ms;
    B.k_s2 = (int32_t) A.k_nb2;
    B.v_s2 = (int32_t) A.v_nb2;
    B.s_gqa = A.n_head / A.n_head_kv;
    B.s_inv_gqa = 1.0f / (float) B.s_gqa;
    if (A.n_head >= DIV_SMALL_MAX || B.s_gqa > 64) HIP_ABORT("attn: %d heads in groups of %d", A.n_head, B.s_gqa);
    return B;
}

void launch_attn_decode(const attn_launch & A_in, hipStream_t st) {
    const attn_launch A = resolve_sources(A_in);
    if (A.n_q < 1 || A.n_q > ATT_DECODE_MAX_Q) HIP_ABORT("attn: n_q %d out of range", A.n_q);
    if (A.rope && A.n_q > ATT_MAX_Q) HIP_ABORT("attn: RoPE folded in for at most %d queries", ATT_MAX_Q);
    if (A.n_head % A.n_head_kv) HIP_ABORT("attn: n_head %% n_head_kv");
    if (A.scratch_bytes < attn_scratch_bytes(A.n_kv, A.n_q, A.n_head, A.hd)) HIP_ABORT("attn: scratch too small");
    if (A.out_q.qs && (A.hd % 32)) HIP_ABORT("attn: quantized output needs hd %% 32 == 0");
    if (A.acc && (A.n_q != 1 || A.out_q.qs || A.out_q8k.qs || ((uintptr_t) A.acc) % 16)) HIP_ABORT("attn: the accumulated output takes one query, no quantized copy, 16-byte alignment");
    if (A.out_q8k.qs && (A.out_q.qs || (A.n_head * A.hd) % 256 || 256 % A.hd)) HIP_ABORT("attn: Q8_K output needs n_head * hd %% 256 == 0 and 256 %% hd == 0");
    if (A.n_q > ATT_MAX_Q) {
        // many queries: scores and PV on the matrix cores
        switch (A.hd) {
            case 64: launch_attn_mq<64>(A, st); break;
            case 96: launch_attn_mq<96>(A, st); break;
            case 128: launch_attn_mq<128>(A, st); break;
            default: HIP_ABORT("attn: unsupported head dim %d", A.hd);
        }
        return;
    }
    switch (A.hd) {
        case 64: launch_attn_hd<64>(A, st); break;
        case 96: launch_attn_hd<96>(A, st); break;
        case 128: launch_attn_hd<128>(A, st); break;
        default: HIP_ABORT("attn: unsupported head dim %d", A.hd);
    }
}

// ---------------------------------------------------------------------------------------------
// Prefill attention: the same chain arithmetic for a batch of queries (n_q > 4), one workgroup per
// (tile of APF_Q queries, head), all of a row's scores held in LDS.
//   scores  K rows staged per 64-position chunk; S[query][pos] from v_mfma_f64_16x16x4f64 over the
//           head dimension (the F16 operands are exact in double, the sum accumulates in double as
//           the chain's), rounded to float, times scale, plus mask. A chunk whose mask is -inf for
//           every query of the tile is not computed: its scores are -inf, as the chain forms them.
//   stats   per row: M = max, e = exp(s - M), S = sum e in double, p = F16(e * (float)(1/S))
//           (flash_attn_ext, p_f32: p = e * (float)(1/S), not rounded to F16).
//   pv      V rows staged per chunk; out[query][dim] from the f64 MFMA over positions with the
//           p (skipped chunks have p = 0 throughout and add nothing), rounded to float.
// (f64 MFMA lane layout as above.)
constexpr int APF_Q = 16;           // queries per workgroup (one MFMA row tile)
constexpr int APF_CHUNK = 64;        // positions per staged K / V chunk (one MFMA column tile per wave)
constexpr int APF_MAX_CHUNKS = 128;  // positions <= 8192

template <int HD>
constexpr int apf_static_lds() {
    return (APF_Q + APF_CHUNK) * (HD + 2) * 2 + APF_MAX_CHUNKS * 4;
}

__host__ __device__ inline int apf_row_stride(int n_kv) {
    return (n_kv + APF_CHUNK - 1) / APF_CHUNK * APF_CHUNK + 4;   // floats; +4 spreads rows over banks
}

template <int HD>
__global__ __launch_bounds__(ATT_THREADS) void attn_prefill_kernel(const attn_launch A) {
    prefetch_kernargs<sizeof(attn_launch)>();
    constexpr int KSTR = HD + 2;     // halves per staged row (one dword of padding)
    constexpr int PIECES = HD / 8;   // 16-byte pieces per row
    __shared__ __half s_q[APF_Q * KSTR];
    __shared__ __half s_kv[APF_CHUNK * KSTR];
    __shared__ int s_live[APF_MAX_CHUNKS];
    __shared__ int s_live_end;       // one past the last live chunk
    extern __shared__ float s_s[];   // [APF_Q][SS]: scores, then e, then p
    // the last query tiles first, every head's before any head's shorter ones (the head is the
    // fastest grid index): under a causal mask they see the most positions, and started last they
    // would leave the chip waiting on a few long workgroups
    const int q0 = (gridDim.y - 1 - blockIdx.y) * APF_Q, h = blockIdx.x;
    const int kvh = h / (A.n_head / A.n_head_kv);
    const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
    const int n_kv = A.n_kv, n_q = A.n_q;
    const int SS = apf_row_stride(n_kv);
    const int n_chunks = (n_kv + APF_CHUNK - 1) / APF_CHUNK;
    const __half * kbase = A.k + (int64_t) kvh * A.k_nb1;
    const __half * vbase = A.v + (int64_t) kvh * A.v_nb1;

    // Q tile rounded to F16 (rows past n_q repeat the last query; their results are not stored)
    for (int i = threadIdx.x; i < APF_Q * HD; i += ATT_THREADS) {
        const int qi = i / HD, d = i % HD;
        const int q = min(q0 + qi, n_q - 1);
        s_q[qi * KSTR + d] = __float2half_rn(A.q[(int64_t) h * A.q_nb1 + (int64_t) q * A.q_nb2 + d]);
    }

    // rows [t0, t0 + nt) of a cache view into registers, and from there into s_kv (zero past nt;
    // with zero_dead, rows masked for every query of the tile also read as zero: skip_masked). The
    // loads are unconditional, at clamped rows, and the zeroing happens at the LDS store: a guarded
    // load, or a register zeroed right after its load, makes the compiler wait for every load.
    static_assert(APF_CHUNK * PIECES % ATT_THREADS == 0, "whole 16-byte pieces per thread");
    constexpr int ITER = APF_CHUNK * PIECES / ATT_THREADS;
    auto load_rows = [&](uint4 (&v)[ITER], const __half * base, int64_t nb_pos, int t0, int nt) {
#pragma unroll
        for (int it = 0; it < ITER; it++) {
            const int pc = threadIdx.x + it * ATT_THREADS;
            const int r = pc / PIECES, c = pc % PIECES;
            v[it] = *(const uint4 *) (base + (int64_t) (t0 + min(r, nt - 1)) * nb_pos + c * 8);
        }
    };
    auto store_rows = [&](uint4 (&v)[ITER], int t0, int nt, bool zero_dead) {
        bool zero[ITER];
#pragma unroll
        for (int it = 0; it < ITER; it++) zero[it] = (threadIdx.x + it * ATT_THREADS) / PIECES >= nt;
        if (zero_dead) {
#pragma unroll
            for (int it = 0; it < ITER; it++) {
                const int r = (threadIdx.x + it * ATT_THREADS) / PIECES;
                bool dead = r < nt;
                for (int q = q0; q < min(q0 + APF_Q, n_q) && dead; q++) dead = mask_at(A, q, t0 + r) == -INFINITY;
                zero[it] = zero[it] || dead;
            }
        }
#pragma unroll
        for (int it = 0; it < ITER; it++) {
            const int pc = threadIdx.x + it * ATT_THREADS;
            const int r = pc / PIECES, c = pc % PIECES;
            uint32_t * d = (uint32_t *) (s_kv + r * KSTR + c * 8);
            const bool z = zero[it];
            d[0] = z ? 0u : v[it].x; d[1] = z ? 0u : v[it].y; d[2] = z ? 0u : v[it].z; d[3] = z ? 0u : v[it].w;
        }
    };
    auto next_live = [&](int ch) {
        while (ch < n_chunks && !s_live[ch]) ch++;
        return ch;
    };

    // the tile's mask rows into s_s (rows past n_q repeat the last query's; 0 without a mask), read
    // once here instead of in every chunk: one position per thread and row at a time, the loads of
    // all APF_Q rows in flight together (unconditional, at clamped positions)
    if (threadIdx.x == 0) s_live_end = 0;
    auto stage_mask = [&](auto load) {
        for (int t0 = 0; t0 < n_kv; t0 += ATT_THREADS) {
            const int t = min(t0 + (int) threadIdx.x, n_kv - 1);
            float v[APF_Q];
#pragma unroll
            for (int qi = 0; qi < APF_Q; qi++) v[qi] = load(min(q0 + qi, n_q - 1), t);
            if (t0 + (int) threadIdx.x < n_kv) {
#pragma unroll
                for (int qi = 0; qi < APF_Q; qi++) s_s[qi * SS + t] = v[qi];
            }
        }
    };
    if (!A.mask) {
        stage_mask([&](int, int) { return 0.0f; });
    } else if (A.mask_f16 && n_kv % 8 == 0 && A.mask_nb1 % 16 == 0 && (uintptr_t) A.mask % 16 == 0) {
        // eight positions per 16-byte load, up to eight loads in flight per thread
        const int per_row = n_kv / 8, total = APF_Q * per_row;
        for (int base = 0; base < total; base += 8 * ATT_THREADS) {
            uint4 v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int i = min(base + u * ATT_THREADS + (int) threadIdx.x, total - 1);
                const int qi = i / per_row, pc = i % per_row;
                v[u] = *(const uint4 *) ((const char *) A.mask + (int64_t) min(q0 + qi, n_q - 1) * A.mask_nb1 + pc * 16);
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int i = base + u * ATT_THREADS + (int) threadIdx.x;
                if (i < total) {
                    const int qi = i / per_row, pc = i % per_row;
                    const uint32_t w[4] = { v[u].x, v[u].y, v[u].z, v[u].w };
                    float f[8];
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float2 x2 = __half22float2(*(const __half2 *) &w[e]);
                        f[2 * e] = x2.x;
                        f[2 * e + 1] = x2.y;
                    }
                    float4 * d = (float4 *) (s_s + qi * SS + pc * 8);
                    d[0] = make_float4(f[0], f[1], f[2], f[3]);
                    d[1] = make_float4(f[4], f[5], f[6], f[7]);
                }
            }
        }
    } else if (A.mask_f16) {
        stage_mask([&](int q, int t) { return __half2float(((const __half *) ((const char *) A.mask + (int64_t) q * A.mask_nb1))[t]); });
    } else {
        stage_mask([&](int q, int t) { return ((const float *) ((const char *) A.mask + (int64_t) q * A.mask_nb1))[t]; });
    }
    __syncthreads();
    // chunk liveness, one wave per chunk (lane = position): a chunk whose mask is -inf for every
    // query of the tile is not computed. Its staged values are then -inf in every row (rows past
    // n_q repeat the last query's), which are the scores the chain forms for it.
    static_assert(APF_CHUNK == WAVE, "one position per lane");
    for (int ch = wave; ch < n_chunks; ch += ATT_WAVES) {
        const int t = ch * APF_CHUNK + lane;
        bool any = !A.mask;
        if (t < n_kv) {
            float v[APF_Q];
#pragma unroll
            for (int qi = 0; qi < APF_Q; qi++) v[qi] = s_s[qi * SS + t];
#pragma unroll
            for (int qi = 0; qi < APF_Q; qi++) any = any || (q0 + qi < n_q && v[qi] != -INFINITY);
        }
        const bool live = __any(any);
        if (lane == 0) {
            s_live[ch] = live;
            if (live) atomicMax(&s_live_end, ch + 1);
        }
    }
    __syncthreads();

    // ---- scores, over the live chunks; wave w takes positions 16 w .. 16 w + 15 of each. The sum
    // over the head dims is exact in any order, so lane group g = lane / 16 takes the NJ consecutive
    // dims NJ g .. NJ g + NJ - 1 (MFMA step j: dim NJ g + j): a lane's K operands are NJ / 8
    // 16-byte pieces of its position's row, loaded straight into registers (no LDS, no barrier),
    // the next live chunk's while this one is used. Q as the A operands, converted once: lane
    // (i + 16 g) holds Q[i][NJ g + j]. ----
    constexpr int NJ = HD / 4;
    constexpr int KU = NJ / 8;                   // 16-byte pieces of a lane's K slice
    static_assert(NJ % 8 == 0, "whole 16-byte K pieces per lane");
    double qd[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) qd[j] = (double) __half2float(s_q[(lane % 16) * KSTR + NJ * (lane / 16) + j]);
    const __half * kslice = kbase + NJ * (lane / 16);
    auto load_k = [&](uint4 (&v)[KU], int c) {
        const int t = min(c * APF_CHUNK + wave * 16 + lane % 16, n_kv - 1);   // clamped, unused past the end
        const uint4 * src = (const uint4 *) (kslice + (int64_t) t * A.k_nb2);
#pragma unroll
        for (int u = 0; u < KU; u++) v[u] = src[u];
    };
    uint4 kc[KU], kn[KU];
    int ch = next_live(0);
    if (ch < n_chunks) load_k(kc, ch);
    while (ch < n_chunks) {
        const int t0 = ch * APF_CHUNK, nt = min(APF_CHUNK, n_kv - t0);
        const int nx = next_live(ch + 1);
        if (nx < n_chunks) load_k(kn, nx);
        // two independent accumulation chains (even and odd steps), added at the end: the double
        // sums are exact for these operands, so the grouping does not matter
        v4d acc = { 0.0, 0.0, 0.0, 0.0 }, acc2 = { 0.0, 0.0, 0.0, 0.0 };
        uint32_t kw[NJ / 2];
        __builtin_memcpy(kw, kc, sizeof(kw));
#pragma unroll
        for (int j = 0; j < NJ; j += 2) {
            const float2 b = __half22float2(*(const __half2 *) &kw[j / 2]);
            acc = __builtin_amdgcn_mfma_f64_16x16x4f64(qd[j], (double) b.x, acc, 0, 0, 0);
            acc2 = __builtin_amdgcn_mfma_f64_16x16x4f64(qd[j + 1], (double) b.y, acc2, 0, 0, 0);
        }
        acc += acc2;
        const int t = wave * 16 + lane % 16;
        if (t < nt) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int qi = lane / 16 + 4 * r;
                float * sp = s_s + qi * SS + t0 + t;
                const float mv = *sp;
                *sp = mv == -INFINITY ? -INFINITY : (float) acc[r] * A.scale + mv;
            }
        }
#pragma unroll
        for (int u = 0; u < KU; u++) kc[u] = kn[u];
        ch = nx;
    }
    __syncthreads();

    // ---- row statistics and probabilities, over the positions before the end of the last live
    // chunk (later ones are -inf, take no part in the sums and are never read again); unrolled so
    // that independent exps interleave ----
    const int n_pos = min(s_live_end * APF_CHUNK, n_kv);
    {
        constexpr int RPW = APF_Q / ATT_WAVES;          // rows qi = wave + 4 k of this wave, together
        float * row[RPW];
        float m[RPW];
#pragma unroll
        for (int k = 0; k < RPW; k++) {
            row[k] = s_s + (wave + ATT_WAVES * k) * SS;
            m[k] = -INFINITY;
        }
        for (int t = lane; t < n_pos; t += WAVE) {
#pragma unroll
            for (int k = 0; k < RPW; k++) m[k] = fmaxf(m[k], row[k][t]);
        }
#pragma unroll
        for (int k = 0; k < RPW; k++) m[k] = wave_max(m[k]);
        double sum[RPW];
#pragma unroll
        for (int k = 0; k < RPW; k++) sum[k] = 0.0;
#pragma unroll 2
        for (int t = lane; t < n_pos; t += WAVE) {
#pragma unroll
            for (int k = 0; k < RPW; k++) {
                // a row masked throughout (m = -inf) gets p = 0
                const float e = m[k] == -INFINITY ? 0.0f : exp_cr(row[k][t] - m[k]);
                row[k][t] = e;
                sum[k] += (double) e;
            }
        }
        float inv[RPW];
#pragma unroll
        for (int k = 0; k < RPW; k++) {
            const double sk = wave_sum_d(sum[k]);
            inv[k] = sk > 0.0 ? (float) (1.0 / sk) : 0.0f;
        }
        for (int t = lane; t < n_pos; t += WAVE) {
#pragma unroll
            for (int k = 0; k < RPW; k++) {
                const float p = as_f32(row[k][t] * inv[k]);
                row[k][t] = A.p_f32 ? p : __half2float(__float2half_rn(p));
            }
        }
    }

    // ---- P V: wave w takes positions 16 w .. 16 w + 15 of every chunk for all HD / 16 output
    // tiles; the four waves' partial sums are added at the end (double sums, exact in practice) ----
    constexpr int NT = HD / 16;                  // 16-dim output tiles
    v4d acc[NT];
#pragma unroll
    for (int k = 0; k < NT; k++) acc[k] = v4d{ 0.0, 0.0, 0.0, 0.0 };
    uint4 kv[ITER];
    ch = next_live(0);
    if (ch < n_chunks) load_rows(kv, vbase, A.v_nb2, ch * APF_CHUNK, min(APF_CHUNK, n_kv - ch * APF_CHUNK));
    while (ch < n_chunks) {
        const int t0 = ch * APF_CHUNK, nt = min(APF_CHUNK, n_kv - t0);
        store_rows(kv, t0, nt, A.skip_masked && A.mask);
        __syncthreads();                         // p of every row and this chunk's V rows visible
        const int nx = next_live(ch + 1);
        if (nx < n_chunks) load_rows(kv, vbase, A.v_nb2, nx * APF_CHUNK, min(APF_CHUNK, n_kv - nx * APF_CHUNK));
#pragma unroll
        for (int s4 = 0; s4 < 4; s4++) {
            const int t = 16 * wave + 4 * s4 + lane / 16;      // rows past nt are staged as zero
            const double a = t < nt ? (double) s_s[(lane % 16) * SS + t0 + t] : 0.0;
#pragma unroll
            for (int k = 0; k < NT; k++) {
                const double b = (double) __half2float(s_kv[t * KSTR + k * 16 + lane % 16]);
                acc[k] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, acc[k], 0, 0, 0);
            }
        }
        __syncthreads();                         // every wave's reads of this chunk's s_kv are done
        ch = nx;
    }
    // register r of lane (c + 16 g) holds row g + 4 r, column c of each tile (the f64 MFMA's D
    // layout); waves 2, 3 hand theirs to waves 0, 1, then wave 1 to wave 0 (the dynamic LDS holds
    // 2 * APF_Q * HD doubles)
    double * red = (double *) s_s;
    auto red_at = [&](int slot, int k, int r) { return red + ((slot * APF_Q + lane / 16 + 4 * r) * HD + k * 16 + lane % 16); };
    if (wave >= 2) {
#pragma unroll
        for (int k = 0; k < NT; k++)
#pragma unroll
            for (int r = 0; r < 4; r++) *red_at(wave - 2, k, r) = acc[k][r];
    }
    __syncthreads();
    if (wave < 2) {
#pragma unroll
        for (int k = 0; k < NT; k++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[k][r] += *red_at(wave, k, r);
    }
    __syncthreads();
    if (wave == 1) {
#pragma unroll
        for (int k = 0; k < NT; k++)
#pragma unroll
            for (int r = 0; r < 4; r++) *red_at(0, k, r) = acc[k][r];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int k = 0; k < NT; k++) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int q = q0 + lane / 16 + 4 * r;
                const double v = acc[k][r] + *red_at(0, k, r);
                if (q < n_q) A.out[(int64_t) q * A.out_nb1 + (int64_t) h * HD + k * 16 + lane % 16] = (float) v;
            }
        }
    }
}

static int max_lds_per_block() {
    static int v = -1;
    if (v < 0) {
        int dev = 0;
        HIP_CHECK(hipGetDevice(&dev));
        HIP_CHECK(hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
    }
    return v;
}

static int apf_static_lds_of(int hd) {
    return hd == 64 ? apf_static_lds<64>() : hd == 96 ? apf_static_lds<96>() : apf_static_lds<128>();
}

int attn_prefill_max_kv(int hd) {
    if (hd != 64 && hd != 96 && hd != 128) return 0;
    const int rows = (max_lds_per_block() - apf_static_lds_of(hd)) / (APF_Q * (int) sizeof(float)) - 4;
    return std::min(rows / APF_CHUNK * APF_CHUNK, APF_MAX_CHUNKS * APF_CHUNK);
}

template <int HD>
static void launch_attn_prefill_hd(const attn_launch & A, hipStream_t st) {
    const size_t lds = std::max((size_t) APF_Q * apf_row_stride(A.n_kv) * sizeof(float), (size_t) 2 * APF_Q * HD * sizeof(double));
    if (lds + apf_static_lds<HD>() > 65536) {
        HIP_CHECK(hipFuncSetAttribute((const void *) attn_prefill_kernel<HD>, hipFuncAttributeMaxDynamicSharedMemorySize, (int) lds));
    }
    launch(attn_prefill_kernel<HD>, dim3(A.n_head, (A.n_q + APF_Q - 1) / APF_Q), dim3(ATT_THREADS), lds, st, A);
}

void launch_attn_prefill(const attn_launch & A, hipStream_t st) {
    if (A.n_q < 1 || A.n_kv < 1 || A.n_kv > attn_prefill_max_kv(A.hd)) HIP_ABORT("attn prefill: n_kv %d out of range", A.n_kv);
    if (A.n_head % A.n_head_kv) HIP_ABORT("attn prefill: n_head %% n_head_kv");
    if (A.out_q.qs) HIP_ABORT("attn prefill: no quantized output");
    if (((uintptr_t) A.k | (uintptr_t) A.v) % 16 || A.k_nb1 % 8 || A.k_nb2 % 8 || A.v_nb1 % 8 || A.v_nb2 % 8) {
        HIP_ABORT("attn prefill: K and V rows must be 16-byte aligned");
    }
    switch (A.hd) {
        case 64: launch_attn_prefill_hd<64>(A, st); break;
        case 96: launch_attn_prefill_hd<96>(A, st); break;
        case 128: launch_attn_prefill_hd<128>(A, st); break;
        default: HIP_ABORT("attn prefill: unsupported head dim %d", A.hd);
    }
}
