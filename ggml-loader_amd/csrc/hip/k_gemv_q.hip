// k_gemv_q.hip — single-column GEMV for Q4_0 / Q8_0 weights (the batch-1 decode hot path).
//
// y[c][r] = W[r] . x[c] (+ add[c][r]) in ggml-cpu's arithmetic: x quantized to Q8_0
// (quantize_row_q8_0), an exact integer dot per 32-element block, the block term formed as ggml
// forms it (Q4_0: (sumi * d_w) * d_x; Q8_0: sumi * (d_w * d_x)) and the terms added in block order,
// so the result is the CPU reference's float.
//
// Mapping: LPR lanes per row (64 / LPR rows per wave); lane l takes blocks l, l + LPR, ... (ITS of
// them, ITS * LPR >= nb), so one load instruction moves LPR consecutive 16-byte block payloads of
// a row. Every weight load of a lane is issued at entry. The block-ordered float sum runs slice by
// slice: slice s (blocks s*LPR .. s*LPR + LPR - 1) is dotted as soon as its loads land, its terms go
// to LDS and the row's first lane adds them to the running sum while the later slices are still in
// flight, so only the last slice's adds follow the last load.
//
// The activation:
//   PRO 0  already quantized (xq / xd / xs); each lane loads its own blocks from memory (L2).
//   PRO 1  rms_norm(x) * w computed in the prologue (ggml's rms_norm -> mul -> quantize_row_q8_0
//          roundings): x and w are read as float4 chunks, each thread holds CPT chunks, the sum of
//          squares is reduced in double (DPP within rows, then across rows and waves in order), and
//          a Q8_0 block is the chunks of 8 consecutive lanes (block max and quant sum by DPP).
//   PRO 2  x quantized as is (the quantization ggml-cpu applies inside mul_mat), same layout.
//   PRO 3  as PRO 2 from doubles (gemv_norm::f64: the decode attention's accumulated output), each
//          rounded to float first; the raw doubles are loaded before the weights and converted after.
// The prologue's loads go out before the weight loads (loads complete in issue order), so the
// prologue runs while the weights stream; the quantized column is staged in LDS.
//
// SwiGLU (gate and up rows of one matrix pair): act = silu(g) * u with the silu and mul ops'
// roundings; with out_q (32 rows per workgroup) the workgroup also writes act's Q8_0 blocks, so
// the down projection reads it pre-quantized.
#include "kernels.h"
#include "gemv_ops.h"

#include "ggml.h"

namespace {

constexpr int QG_MAX_WAVES = 16;

__host__ __device__ constexpr int qg_term_stride(int lpr) { return lpr + 4; }

// dynamic LDS: [terms: rows_pb * NCH][TS] floats | [xq: K] | [xd: nb] | [xs: nb] | [red: 16 doubles]
// | [act: rows_pb floats]
struct qg_lds {
    float *   terms;
    int8_t *  xq;
    float *   xd;
    int32_t * xs;
    double *  red;
    float *   act;
};

__host__ __device__ inline size_t qg_lds_bytes(int lpr, int rows_pb, int nch, int K, bool staged) {
    size_t b = (size_t) rows_pb * nch * qg_term_stride(lpr) * 4;
    if (staged) b += (size_t) K + (size_t) (K / 32) * 8;
    b = (b + 15) & ~(size_t) 15;
    b += QG_MAX_WAVES * 8;
    b += (size_t) rows_pb * 4;
    return b;
}

__device__ __forceinline__ qg_lds qg_layout(uint8_t * smem, int lpr, int rows_pb, int nch, int K, bool staged) {
    qg_lds s;
    s.terms = (float *) smem;
    size_t off = (size_t) rows_pb * nch * qg_term_stride(lpr) * 4;
    s.xq = (int8_t *) (smem + off);
    if (staged) off += (size_t) K;
    s.xd = (float *) (smem + off);
    if (staged) off += (size_t) (K / 32) * 4;
    s.xs = (int32_t *) (smem + off);
    if (staged) off += (size_t) (K / 32) * 4;
    off = (off + 15) & ~(size_t) 15;
    s.red = (double *) (smem + off);
    off += QG_MAX_WAVES * 8;
    s.act = (float *) (smem + off);
    return s;
}

// Q8_0 quantization of 4 consecutive values held by one lane, 8 consecutive lanes per 32-element
// block (quantize_row_q8_0_ref: d = amax / 127, q = roundf(v * (d ? 1/d : 0)), d kept as fp16);
// returns the packed bytes, the block's d and the block's quant sum (every lane of the group).
__device__ __forceinline__ int q8_quant4(float v0, float v1, float v2, float v3, float & dd_out, int & sum_out) {
    const float amax = max8_dpp(fmaxf(fmaxf(fabsf(v0), fabsf(v1)), fmaxf(fabsf(v2), fabsf(v3))));
    const float dd = amax / 127;
    const float id = dd ? 1.0f / dd : 0.0f;
    const int q0 = (int) roundf(v0 * id), q1 = (int) roundf(v1 * id), q2 = (int) roundf(v2 * id), q3 = (int) roundf(v3 * id);
    sum_out = sum8_dpp(q0 + q1 + q2 + q3);
    dd_out = __half2float(__float2half_rn(dd));
    return (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | ((q3 & 0xff) << 24);
}

template <int TYPE, int LPR, int ITS, bool SWIGLU, int PRO, int CPT, int MAXT>
__global__ __launch_bounds__(MAXT) void gemv_q_kernel(const gemv_kargs a) {
    prefetch_kernargs<sizeof(gemv_kargs)>();
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int RPW = WAVE / LPR;
    constexpr int NCH = SWIGLU ? 2 : 1;
    constexpr int QS = TYPE == GGML_TYPE_Q4_0 ? Q4_0_QS : Q8_0_QS;
    constexpr int TS = qg_term_stride(LPR);
    const gemv_launch & L = a.L;
    const int t = threadIdx.x, nt = blockDim.x;
    const int lane = t % WAVE, wave = t / WAVE;
    const int g = lane / LPR, l = lane % LPR;
    const int rows_pb = a.rows_per_block;
    const int rib = wave * RPW + g;
    const int row = blockIdx.x * rows_pb + rib;
    const int col = blockIdx.y;
    const int K = L.K, nb = K / 32, nc = K / 4;
    const int mi = SWIGLU ? 0 : find_mat(a, blockIdx.x * rows_pb);   // uniform: the workgroup's matrix
    const int lrow = SWIGLU ? row : row - a.row_begin[mi];
    const bool valid = row < a.total_rows && lrow < L.m[mi].n_rows;
    const qg_lds s = qg_layout(smem, LPR, rows_pb, NCH, K, PRO != 0);

    // mul_mat_id: the expert of this column and its activation column
    int xcol = col;
    int64_t erow = 0;
    if (L.ids) {
        const int tk = col / L.n_slots, sl = col % L.n_slots;
        xcol = tk * L.x_cols + sl % L.x_cols;
        const int e = min(max(L.ids[(int64_t) tk * L.ids_stride + sl], 0), L.n_experts - 1);
        erow = (int64_t) e * L.expert_rows;
    }

    // ---- prologue loads (before the weights): CPT float4 chunks of x (and of the norm weight) ----
    float4 xv[CPT], wv[CPT];
    double2 xlo[PRO == 3 ? CPT : 1], xhi[PRO == 3 ? CPT : 1];
    if constexpr (PRO == 3) {
        const double2 * x2 = (const double2 *) ((const double *) L.norm.x + (int64_t) xcol * L.norm.x_stride);
#pragma unroll
        for (int k = 0; k < CPT; k++) {
            const int c = wrap_index(t + k * nt, nc, t);
            xlo[k] = x2[2 * c];
            xhi[k] = x2[2 * c + 1];
        }
        asm volatile("" ::: "memory");   // these loads stay ahead of the weights'
    } else if constexpr (PRO != 0) {
        const float4 * x4 = (const float4 *) (L.norm.x + (int64_t) xcol * L.norm.x_stride);
        const float4 * w4 = (const float4 *) (PRO == 1 && L.norm.w ? L.norm.w : L.norm.x);
#pragma unroll
        for (int k = 0; k < CPT; k++) {
            const int c = wrap_index(t + k * nt, nc, t);
            xv[k] = x4[c];
            if (PRO == 1) wv[k] = w4[c];
        }
    }
    // The rms norm's per-thread sum of squares is formed before any weight load goes out: its x
    // loads then return from an idle memory system (behind the weight loads of every workgroup they
    // waited about 3 us), and the weights stream while the sum is reduced and x quantized.
    double ss = 0.0;
    if constexpr (PRO == 1) {
#pragma unroll
        for (int k = 0; k < CPT; k++) {
            if (t + k * nt < nc) {
                ss += (double) (xv[k].x * xv[k].x);
                ss += (double) (xv[k].y * xv[k].y);
                ss += (double) (xv[k].z * xv[k].z);
                ss += (double) (xv[k].w * xv[k].w);
            }
        }
        asm volatile("" ::"v"(ss) : "memory");
    }

    // ---- every weight load of this lane (row and block clamped into the matrix) ----
    uint4 qa[NCH][ITS], qb[NCH][ITS];
    unsigned short dw[NCH][ITS];
#pragma unroll
    for (int ch = 0; ch < NCH; ch++) {
        const gemv_mat & wm = L.m[SWIGLU ? ch : mi];
        const int64_t wr = erow + min(lrow, wm.n_rows - 1);
        const uint8_t * wq = wm.w + wr * nb * QS;
        const unsigned short * wd = (const unsigned short *) wm.wd + wr * nb;
#pragma unroll
        for (int it = 0; it < ITS; it++) {
            const int b = min(l + it * LPR, nb - 1);
            qa[ch][it] = *(const uint4 *) (wq + (int64_t) b * QS);
            if (TYPE == GGML_TYPE_Q8_0) qb[ch][it] = *(const uint4 *) (wq + (int64_t) b * QS + 16);
            dw[ch][it] = wd[b];
        }
    }

    // the raw doubles are converted only after every weight load is out (converted earlier, the
    // wait for them would hold back the weight loads still to issue)
    if constexpr (PRO == 3) __builtin_amdgcn_sched_barrier(0);
    // ---- the activation blocks this lane dots ----
    int4 xa[ITS], xb[ITS];
    float xd[ITS];
    int xs[ITS];
    if constexpr (PRO == 0) {
        const int8_t * xq = L.xq + (int64_t) xcol * K;
#pragma unroll
        for (int it = 0; it < ITS; it++) {
            const int b = min(l + it * LPR, nb - 1);
            xa[it] = *(const int4 *) (xq + b * 32);
            xb[it] = *(const int4 *) (xq + b * 32 + 16);
            xd[it] = L.xd[(int64_t) xcol * nb + b];
            xs[it] = L.xs[(int64_t) xcol * nb + b];
        }
    } else {
        float scale = 1.0f;
        if constexpr (PRO == 1) {
            ss = wave_sum_d_dpp(ss);
            if (lane == 0) s.red[wave] = ss;
            __syncthreads();
            double tot = 0.0;
            for (int w = 0; w < nt / WAVE; w++) tot += s.red[w];
            const float mean = (float) (tot / (double) K);
            scale = 1.0f / sqrtf(mean + L.norm.eps);
        }
#pragma unroll
        for (int k = 0; k < CPT; k++) {
            const int c = t + k * nt;                 // chunk c: elements 4c .. 4c + 3 of block c / 8
            if constexpr (PRO == 3) xv[k] = make_float4((float) xlo[k].x, (float) xlo[k].y, (float) xhi[k].x, (float) xhi[k].y);
            float v0 = xv[k].x, v1 = xv[k].y, v2 = xv[k].z, v3 = xv[k].w;
            if (PRO == 1) {
                v0 = v0 * scale; v1 = v1 * scale; v2 = v2 * scale; v3 = v3 * scale;
                if (L.norm.w) { v0 = v0 * wv[k].x; v1 = v1 * wv[k].y; v2 = v2 * wv[k].z; v3 = v3 * wv[k].w; }
            }
            float dd;
            int sum;
            const int packed = q8_quant4(v0, v1, v2, v3, dd, sum);
            if (c < nc) {
                ((int *) s.xq)[c] = packed;
                if ((t % 8) == 0) {
                    s.xd[c / 8] = dd;
                    s.xs[c / 8] = sum;
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int it = 0; it < ITS; it++) {
            const int b = min(l + it * LPR, nb - 1);
            xa[it] = *(const int4 *) (s.xq + b * 32);
            xb[it] = *(const int4 *) (s.xq + b * 32 + 16);
            xd[it] = s.xd[b];
            xs[it] = s.xs[b];
        }
    }

    // ---- dots and the block-ordered sums, one slice at a time ----
    float * tr = s.terms + rib * NCH * TS;
    float acc = 0.0f;
#pragma unroll
    for (int it = 0; it < ITS; it++) {
        const int b = l + it * LPR;
#pragma unroll
        for (int ch = 0; ch < NCH; ch++) {
            const float dwf = __half2float(__ushort_as_half(dw[ch][it]));
            float term;
            if (TYPE == GGML_TYPE_Q4_0) {
                const int sumi = dot_q4_0_block(qa[ch][it], xa[it], xb[it]) - 8 * xs[it];
                term = ((float) sumi * dwf) * xd[it];          // ggml: sumi*d_x*d_y
            } else {
                const int sumi = dot_q8_0_block(qa[ch][it], qb[ch][it], xa[it], xb[it]);
                term = (float) sumi * (dwf * xd[it]);          // ggml: sumi*(d_x*d_y)
            }
            tr[ch * TS + l] = b < nb ? term : 0.0f;
        }
        // the slice's terms were written by lanes of this wave: a wave-level ordering point
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int n = min(LPR, nb - it * LPR);
        if (l < NCH) {
            const float * tp = tr + l * TS;            // lane 0: the gate (or only) chain, lane 1: up
            if (n == LPR) {
#pragma unroll
                for (int k = 0; k < LPR / 4; k++) {
                    const float4 v4 = ((const float4 *) tp)[k];
                    acc = acc + v4.x + v4.y + v4.z + v4.w;
                }
            } else {
                for (int k = 0; k < n; k++) acc = acc + tp[k];
            }
        }
        if (it + 1 < ITS) {
            // the next slice overwrites the terms: every lane's reads of this one come first
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    }

    if constexpr (SWIGLU) {
        // act = silu(gate) * up (two roundings, as the silu and mul ops); up sits on the next lane
        const float uv = __shfl_down(acc, 1, WAVE);
        const float sl = acc / (1.0f + exp_cr(-acc));
        const float act = sl * uv;
        if (valid && l == 0) L.m[0].y[(int64_t) col * L.m[0].y_stride + row] = act;
        if (L.out_q.qs) {
            // the workgroup's rows (a multiple of 32) quantized to Q8_0: 4 rows per thread, 8 threads
            // per block
            if (l == 0) s.act[rib] = valid ? act : 0.0f;
            __syncthreads();
            if (t < rows_pb / 4) {
                const float4 v = ((const float4 *) s.act)[t];
                float dd;
                int sum;
                const int packed = q8_quant4(v.x, v.y, v.z, v.w, dd, sum);
                const int r0 = blockIdx.x * rows_pb + 4 * t;
                const int nr = L.m[0].n_rows;
                if (r0 < nr) {
                    ((int *) (L.out_q.qs + (int64_t) col * nr))[r0 / 4] = packed;
                    if ((t % 8) == 0) {
                        L.out_q.d[(int64_t) col * (nr / 32) + r0 / 32] = dd;
                        L.out_q.s[(int64_t) col * (nr / 32) + r0 / 32] = sum;
                    }
                }
            }
        }
    } else {
        if (valid && l == 0) {
            const gemv_mat & m = L.m[mi];
            float v = acc;
            if (m.add) v = v + m.add[(int64_t) col * m.add_stride + lrow];
            m.y[(int64_t) col * m.y_stride + lrow] = v;
        }
    }
}

// ---- host: shapes ----

struct qg_shape {
    int lpr, its, waves, cpt;
};

// slices per lane, rounded up to an instantiated count
int qg_its_of(int nb, int lpr) {
    const int its = (nb + lpr - 1) / lpr;
    if (its <= 4) return its;
    if (its <= 6) return 6;
    if (its <= 8) return 8;
    return -1;
}

// Threads per workgroup (the register budget): 256 for a plain launch, 512 with a prologue or
// SwiGLU, 1024 for the 32-row SwiGLU launches that quantize act (slices <= 4)
template <int TYPE, int LPR, int ITS, bool SWIGLU, int PRO, int CPT>
void qg_launch_t(const gemv_kargs & ka, int waves, size_t lds, hipStream_t st) {
    const dim3 grid((ka.total_rows + ka.rows_per_block - 1) / ka.rows_per_block, ka.L.ncols);
    const dim3 block(waves * WAVE);
    if constexpr (SWIGLU) {
        if (waves > 8) {
            if constexpr (ITS <= 4) return launch((gemv_q_kernel<TYPE, LPR, ITS, SWIGLU, PRO, CPT, 1024>), grid, block, lds, st, ka);
            HIP_ABORT("gemv: %d waves per workgroup", waves);
        }
        launch((gemv_q_kernel<TYPE, LPR, ITS, SWIGLU, PRO, CPT, 512>), grid, block, lds, st, ka);
    } else if constexpr (PRO != 0) {
        if (waves > 8) HIP_ABORT("gemv: %d waves per workgroup", waves);
        launch((gemv_q_kernel<TYPE, LPR, ITS, SWIGLU, PRO, CPT, 512>), grid, block, lds, st, ka);
    } else {
        if (waves > 4) HIP_ABORT("gemv: %d waves per workgroup", waves);
        launch((gemv_q_kernel<TYPE, LPR, ITS, SWIGLU, PRO, CPT, 256>), grid, block, lds, st, ka);
    }
}

template <int TYPE, int LPR, int ITS, bool SWIGLU>
void qg_launch_its(const gemv_kargs & ka, int pro, int waves, int cpt, size_t lds, hipStream_t st) {
    if (pro == 0) {
        qg_launch_t<TYPE, LPR, ITS, SWIGLU, 0, 1>(ka, waves, lds, st);
    } else if (pro == 1) {
        if (cpt == 1) qg_launch_t<TYPE, LPR, ITS, SWIGLU, 1, 1>(ka, waves, lds, st);
        else qg_launch_t<TYPE, LPR, ITS, SWIGLU, 1, 2>(ka, waves, lds, st);
    } else if (pro == 2 || SWIGLU) {
        if (cpt == 1) qg_launch_t<TYPE, LPR, ITS, SWIGLU, 2, 1>(ka, waves, lds, st);
        else if (cpt == 2) qg_launch_t<TYPE, LPR, ITS, SWIGLU, 2, 2>(ka, waves, lds, st);
        else qg_launch_t<TYPE, LPR, ITS, SWIGLU, 2, 4>(ka, waves, lds, st);
    } else if constexpr (!SWIGLU) {
        if (cpt == 1) qg_launch_t<TYPE, LPR, ITS, false, 3, 1>(ka, waves, lds, st);
        else if (cpt == 2) qg_launch_t<TYPE, LPR, ITS, false, 3, 2>(ka, waves, lds, st);
        else qg_launch_t<TYPE, LPR, ITS, false, 3, 4>(ka, waves, lds, st);
    }
}

template <int TYPE, bool SWIGLU>
void qg_dispatch(const gemv_kargs & ka, const qg_shape & sh, int pro, size_t lds, hipStream_t st) {
#define QG_CASE(LPR_, ITS_) \
    if (sh.lpr == LPR_ && sh.its == ITS_) return qg_launch_its<TYPE, LPR_, ITS_, SWIGLU>(ka, pro, sh.waves, sh.cpt, lds, st);
    QG_CASE(16, 1)
    QG_CASE(32, 1) QG_CASE(32, 2) QG_CASE(32, 3) QG_CASE(32, 4) QG_CASE(32, 6) QG_CASE(32, 8)
    if constexpr (!SWIGLU) {
        QG_CASE(64, 6) QG_CASE(64, 8)
    }
#undef QG_CASE
    HIP_ABORT("gemv: no kernel for %d lanes per row x %d slices", sh.lpr, sh.its);
}

}  // namespace

// Whether the single-column kernel takes this launch (Q4_0 / Q8_0 weights, rows up to 16384 blocks
// of 32, a prologue the chunks per thread can hold)
bool gemv_q_supported(const gemv_launch & L) {
    if (L.type != GGML_TYPE_Q4_0 && L.type != GGML_TYPE_Q8_0) return false;
    if (L.K % 128 || L.K > GEMV_MAX_K) return false;
    if (L.swiglu && L.K > gemv_swiglu_max_k(L.type)) return false;
    return true;
}

void launch_gemv_q(const gemv_launch & L, hipStream_t st) {
    gemv_kargs ka;
    ka.L = L;
    const int nb = L.K / 32, nc = L.K / 4;
    const int pro = !L.norm.x ? 0 : L.norm.f64 ? 3 : L.norm.rms ? 1 : 2;
    if (pro == 3 && (L.swiglu || L.norm.rms || L.norm.x_stride % 2)) HIP_ABORT("gemv: a double-valued column is quantized as is, without SwiGLU");
    const bool epq = L.swiglu && L.out_q.qs;
    if (epq && L.m[0].n_rows % 32) HIP_ABORT("gemv: quantized SwiGLU output needs rows %% 32 == 0");
    qg_shape sh{};
    // lanes per row: 32 for rows of 17..256 blocks (slices of 32 blocks; 1..8 of them), 16 for
    // shorter rows, 64 for longer ones
    sh.lpr = nb <= 16 ? 16 : nb <= 256 ? 32 : 64;
    if (L.swiglu && sh.lpr == 64) sh.lpr = 32;
    sh.its = qg_its_of(nb, sh.lpr);
    if (sh.its < 0) HIP_ABORT("gemv: K=%d too long", L.K);
    const int rpw = WAVE / sh.lpr;
    if (epq) {
        if (L.K > GEMV_SWIGLU_QOUT_MAX_K) HIP_ABORT("gemv: quantized SwiGLU output with K=%d", L.K);
        sh.waves = 32 / rpw;                       // 32 rows per workgroup
    } else if (pro == 0) {
        sh.waves = 4;
    } else {
        // enough threads for the prologue's chunks in at most 2 (rms) or 4 (quantize only) per thread
        const int cmax = pro == 1 ? 2 : 4;
        sh.waves = std::max(4, (nc + cmax * WAVE - 1) / (cmax * WAVE));
        if (sh.waves > 8) HIP_ABORT("gemv: K=%d too long for the activation prologue", L.K);
    }
    if (pro != 0) {
        const int need = (nc + sh.waves * WAVE - 1) / (sh.waves * WAVE);
        const int cmax = pro == 1 ? 2 : 4;
        if (need > cmax) HIP_ABORT("gemv: K=%d too long for the activation prologue", L.K);
        sh.cpt = pro == 1 ? need : (need <= 1 ? 1 : need <= 2 ? 2 : 4);
    } else {
        sh.cpt = 1;
    }
    ka.rows_per_block = sh.waves * rpw;
    int r = 0;
    if (L.swiglu) {
        if (L.n_mats != 2 || L.m[0].n_rows != L.m[1].n_rows) HIP_ABORT("gemv: swiglu needs two equal matrices");
        for (int i = 0; i <= GEMV_MAX_MATS; i++) ka.row_begin[i] = 0;
        ka.total_rows = L.m[0].n_rows;
    } else {
        // every matrix starts on a workgroup boundary
        for (int i = 0; i < L.n_mats; i++) {
            ka.row_begin[i] = r;
            r += (L.m[i].n_rows + ka.rows_per_block - 1) / ka.rows_per_block * ka.rows_per_block;
        }
        for (int i = L.n_mats; i <= GEMV_MAX_MATS; i++) ka.row_begin[i] = r;
        ka.total_rows = r;
    }
    const size_t lds = qg_lds_bytes(sh.lpr, ka.rows_per_block, L.swiglu ? 2 : 1, L.K, pro != 0);
    if (lds > 64 * 1024) HIP_ABORT("gemv: K=%d needs %zu bytes of LDS", L.K, lds);
    if (L.type == GGML_TYPE_Q4_0) {
        if (L.swiglu) qg_dispatch<GGML_TYPE_Q4_0, true>(ka, sh, pro, lds, st);
        else qg_dispatch<GGML_TYPE_Q4_0, false>(ka, sh, pro, lds, st);
    } else {
        if (L.swiglu) qg_dispatch<GGML_TYPE_Q8_0, true>(ka, sh, pro, lds, st);
        else qg_dispatch<GGML_TYPE_Q8_0, false>(ka, sh, pro, lds, st);
    }
}
