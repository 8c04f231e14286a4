// k_ops.hip — normalization, element-wise, RoPE, softmax, copies, row gathers and the generic
// (non-quantized) mul_mat used off the fused decode path. Arithmetic follows the ggml op
// semantics the graph encodes (reference model.cpp:1071-1474): RMSNorm sums x*x in double and
// scales by 1/sqrtf(mean + eps) before the weight multiply; RoPE iterates theta *= theta_scale
// in float from theta = pos; softmax exponentiates w - max with the sum kept in double.
#include "kernels.h"
#include "tview_ops.h"

#include "ggml.h"

// ---------------------------------------------------------------------------------------------
// typed element access

static int64_t nelem(const tview & t) { return t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3]; }

static unsigned grid1(int64_t n, int threads) { return (unsigned) ((n + threads - 1) / threads); }

// ---------------------------------------------------------------------------------------------
// RMSNorm (+ weight multiply, + activation quantization)

// Q8_K quantization (ggml quantize_row_q8_K_ref) of one 256-element super-block held one value per
// thread of a 256-thread block: the value of largest magnitude (lowest index on ties) sets
// iscale = -127 / max, q = min(127, round-half-even(iscale * o)), d = 1 / iscale (0 for an all-zero
// block), bsums = sums of 16 consecutive q. qs, d and bsums point at the super-block's entries.
// Every thread of the block must call it (it synchronizes the block).
__device__ void q8k_superblock(float o, int t, int8_t * qs, float * d, int16_t * bsums) {
    __shared__ float s_fx[4];
    __shared__ int s_ix[4];
    __shared__ float s_vx[4];
    float ax = fabsf(o);
    int idx = t;
    float val = o;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ax2 = __shfl_xor(ax, off, WAVE);
        const int idx2 = __shfl_xor(idx, off, WAVE);
        const float val2 = __shfl_xor(val, off, WAVE);
        if (ax2 > ax || (ax2 == ax && idx2 < idx)) { ax = ax2; idx = idx2; val = val2; }
    }
    __syncthreads();
    if ((t % 64) == 0) { s_fx[t / 64] = ax; s_ix[t / 64] = idx; s_vx[t / 64] = val; }
    __syncthreads();
    float bax = s_fx[0], bval = s_vx[0];
    int bidx = s_ix[0];
    for (int wv = 1; wv < 4; wv++) {
        if (s_fx[wv] > bax || (s_fx[wv] == bax && s_ix[wv] < bidx)) { bax = s_fx[wv]; bidx = s_ix[wv]; bval = s_vx[wv]; }
    }
    int q = 0;
    if (bax != 0.0f) {
        const float iscale = -127.f / bval;
        q = round_half_even(iscale * o);
        q = q < 127 ? q : 127;
        if (t == 0) *d = 1 / iscale;
    } else if (t == 0) {
        *d = 0.0f;
    }
    qs[t] = (int8_t) q;
    const float bs = group_sum<16>((float) q);
    if ((t % 16) == 0) bsums[t / 16] = (int16_t) bs;
}

// One 256-thread block per row; each thread holds its EPT elements (i = it*256 + t) in registers,
// so the row is read once with every load issued up front.
template <int QUANT, int EPT> // QUANT: 0 none, 1 Q8_0 (32-blocks), 2 Q8_K (256-blocks)
__global__ __launch_bounds__(256) void rms_norm_kernel(const float * __restrict__ x, int64_t x_stride,
        const float * __restrict__ w, float * __restrict__ y, int64_t y_stride, int64_t n, float eps,
        q8_act q8, q8k_act q8k) {
    __shared__ double s_part[4];
    const int64_t row = blockIdx.x;
    const float * xr = x + row * x_stride;
    float * yr = y + row * y_stride;
    const int t = threadIdx.x;
    float v[EPT];
#pragma unroll
    for (int it = 0; it < EPT; it++) {
        const int64_t i = (int64_t) it * 256 + t;
        v[it] = i < n ? xr[i] : 0.0f;
    }
    double sum = 0.0;
#pragma unroll
    for (int it = 0; it < EPT; it++) sum += (double) (v[it] * v[it]);
    sum = wave_sum_d(sum);
    if ((t % 64) == 0) s_part[t / 64] = sum;
    __syncthreads();
    const double total = s_part[0] + s_part[1] + s_part[2] + s_part[3];
    const float mean = (float) (total / (double) n);
    const float scale = 1.0f / sqrtf(mean + eps);
#pragma unroll
    for (int it = 0; it < EPT; it++) {
        const int64_t i = (int64_t) it * 256 + t;
        if ((int64_t) it * 256 >= n) break;       // uniform
        float o = 0.0f;
        if (i < n) {
            o = v[it] * scale;
            if (w) o = o * w[i];
            yr[i] = o;
        }
        if (QUANT == 1) {
            // 32 consecutive elements live in 32 consecutive lanes
            const float amax = group_max<32>(fabsf(o));
            const float dd = amax / 127;
            const float id = dd ? 1.0f / dd : 0.0f;
            const int q = (int) roundf(o * id);
            const float qsum = group_sum<32>((float) q);
            if (i < n) {
                q8.qs[row * n + i] = (int8_t) q;
                if ((i % 32) == 0) {
                    q8.d[row * (n / 32) + i / 32] = __half2float(__float2half_rn(dd));
                    q8.s[row * (n / 32) + i / 32] = (int32_t) qsum;
                }
            }
        } else if (QUANT == 2) {
            // one super-block of 256 per iteration (n % 256 == 0)
            q8k_superblock(o, t, q8k.qs + row * n + (int64_t) it * 256, q8k.d + row * (n / 256) + it,
                           q8k.bsums + row * (n / 16) + (int64_t) it * 16);
        }
    }
}

template <int QUANT>
static void launch_rms_norm_q(const float * x, int64_t x_stride, const float * w, float * y, int64_t y_stride,
                              int64_t n, int64_t ncols, float eps, q8_act a, q8k_act b, hipStream_t st) {
    const int64_t ept = (n + 255) / 256;
    dim3 grid((unsigned) ncols), blk(256);
    if (ept <= 1) launch((rms_norm_kernel<QUANT, 1>), grid, blk, 0, st, x, x_stride, w, y, y_stride, n, eps, a, b);
    else if (ept <= 2) launch((rms_norm_kernel<QUANT, 2>), grid, blk, 0, st, x, x_stride, w, y, y_stride, n, eps, a, b);
    else if (ept <= 4) launch((rms_norm_kernel<QUANT, 4>), grid, blk, 0, st, x, x_stride, w, y, y_stride, n, eps, a, b);
    else if (ept <= 8) launch((rms_norm_kernel<QUANT, 8>), grid, blk, 0, st, x, x_stride, w, y, y_stride, n, eps, a, b);
    else if (ept <= 16) launch((rms_norm_kernel<QUANT, 16>), grid, blk, 0, st, x, x_stride, w, y, y_stride, n, eps, a, b);
    else if (ept <= 32) launch((rms_norm_kernel<QUANT, 32>), grid, blk, 0, st, x, x_stride, w, y, y_stride, n, eps, a, b);
    else HIP_ABORT("rms_norm: rows of %lld elements are not supported", (long long) n);
}

void launch_rms_norm(const float * x, int64_t x_stride, const float * w, float * y, int64_t y_stride,
                     int64_t n, int64_t ncols, float eps, const q8_act * q8, const q8k_act * q8k, hipStream_t st) {
    q8_act a{};
    q8k_act b{};
    if (q8) {
        if (n % 32) HIP_ABORT("rms_norm: q8 output needs n %% 32 == 0");
        launch_rms_norm_q<1>(x, x_stride, w, y, y_stride, n, ncols, eps, *q8, b, st);
    } else if (q8k) {
        if (n % 256) HIP_ABORT("rms_norm: q8K output needs n %% 256 == 0");
        launch_rms_norm_q<2>(x, x_stride, w, y, y_stride, n, ncols, eps, a, *q8k, st);
    } else {
        launch_rms_norm_q<0>(x, x_stride, w, y, y_stride, n, ncols, eps, a, b, st);
    }
}

// generic strided: one block per row (i1, i2, i3)
__global__ __launch_bounds__(256) void rms_norm_strided_kernel(tview x, tview y, float eps) {
    __shared__ double s_part[4];
    const int64_t r = blockIdx.x;
    const int64_t i1 = r % x.ne[1], i2 = (r / x.ne[1]) % x.ne[2], i3 = r / (x.ne[1] * x.ne[2]);
    const int t = threadIdx.x;
    double sum = 0.0;
    for (int64_t i = t; i < x.ne[0]; i += 256) {
        const float v = *(const float *) at(x, i, i1, i2, i3);
        sum += (double) (v * v);
    }
    sum = wave_sum_d(sum);
    if ((t % 64) == 0) s_part[t / 64] = sum;
    __syncthreads();
    const double total = s_part[0] + s_part[1] + s_part[2] + s_part[3];
    const float mean = (float) (total / (double) x.ne[0]);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int64_t i = t; i < x.ne[0]; i += 256) {
        *(float *) at(y, i, i1, i2, i3) = *(const float *) at(x, i, i1, i2, i3) * scale;
    }
}

void launch_rms_norm_strided(const tview & x, const tview & y, float eps, hipStream_t st) {
    const int64_t rows = x.ne[1] * x.ne[2] * x.ne[3];
    launch(rms_norm_strided_kernel, dim3((unsigned) rows), dim3(256), 0, st, x, y, eps);
}

// ---------------------------------------------------------------------------------------------
// element-wise

__global__ void binary_kernel(int op, tview a, tview b, tview d, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const idx4 k = unflatten(i, d.ne);
    const float x = ld(at(a, k.i0, k.i1, k.i2, k.i3), a.type);
    const float y = ld(at(b, k.i0 % b.ne[0], k.i1 % b.ne[1], k.i2 % b.ne[2], k.i3 % b.ne[3]), b.type);
    st(at(d, k.i0, k.i1, k.i2, k.i3), d.type, op == 0 ? x + y : op == 1 ? x * y : op == 3 ? x - y : x / y);
}

void launch_binary(int op, const tview & a, const tview & b, const tview & dst, hipStream_t st) {
    const int64_t n = nelem(dst);
    if (n == 0) return;
    launch(binary_kernel, dim3(grid1(n, 256)), dim3(256), 0, st, op, a, b, dst, n);
}

// ---------------------------------------------------------------------------------------------
// MoE routing and expert combination

// one wave per row: the row sum accumulated in double (ggml's generic row sum)
__global__ void sum_rows_kernel(tview a, tview d, int64_t rows) {
    const int64_t r = (int64_t) blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE;
    const int lane = threadIdx.x % WAVE;
    if (r >= rows) return;
    const int64_t i1 = r % a.ne[1], i2 = (r / a.ne[1]) % a.ne[2], i3 = r / (a.ne[1] * a.ne[2]);
    double sum = 0.0;
    for (int64_t i0 = lane; i0 < a.ne[0]; i0 += WAVE) sum += (double) ld(at(a, i0, i1, i2, i3), a.type);
    sum = wave_sum_d(sum);
    if (lane == 0) st(at(d, 0, i1, i2, i3), d.type, (float) sum);
}

void launch_sum_rows(const tview & a, const tview & dst, hipStream_t st) {
    const int64_t rows = a.ne[1] * a.ne[2] * a.ne[3];
    if (rows == 0) return;
    launch(sum_rows_kernel, dim3(grid1(rows, 4)), dim3(256), 0, st, a, dst, rows);
}

// one workgroup per row: element i goes to position rank(i) = the number of elements ordered before
// it, where equal values order by ascending index (a stable sort; the router's tie rule)
__global__ __launch_bounds__(256) void argsort_kernel(tview a, tview d, int desc) {
    extern __shared__ float s_row[];
    const int64_t r = blockIdx.x;
    const int64_t i1 = r % a.ne[1], i2 = (r / a.ne[1]) % a.ne[2], i3 = r / (a.ne[1] * a.ne[2]);
    const int n = (int) a.ne[0];
    for (int i = threadIdx.x; i < n; i += blockDim.x) s_row[i] = ld(at(a, i, i1, i2, i3), a.type);
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = s_row[i];
        int rank = 0;
        for (int j = 0; j < n; j++) {
            const float u = s_row[j];
            rank += (desc ? u > v : u < v) || (u == v && j < i);
        }
        *(int32_t *) at(d, rank, i1, i2, i3) = i;
    }
}

void launch_argsort(const tview & a, const tview & dst, bool desc, hipStream_t st) {
    const int64_t rows = a.ne[1] * a.ne[2] * a.ne[3];
    if (a.ne[0] > ARGSORT_MAX_ROW) HIP_ABORT("argsort: rows of %lld exceed %d", (long long) a.ne[0], ARGSORT_MAX_ROW);
    if (rows == 0) return;
    launch(argsort_kernel, dim3((unsigned) rows), dim3(256), (size_t) a.ne[0] * sizeof(float), st, a, dst, desc ? 1 : 0);
}

// out[:, t] = ((e[:, 0, t] * w[0, t] + e[:, 1, t] * w[1, t]) + ...) (+ res[:, t]): the graph's
// mul by the routing weights, its chain of adds over the slots in order, and the residual add
// Up to WS_BATCH slots' values are loaded together before the sum (a loop of load -> use would put
// one round trip per slot on the path); the products are added in slot order as before.
constexpr int WS_BATCH = 8;
__global__ void moe_wsum_kernel(moe_wsum M) {
    prefetch_kernargs<sizeof(moe_wsum)>();
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t t = blockIdx.y;
    if (i >= M.n_embd) return;
    const float * e = M.e + t * M.e_nb2 + i;
    const float * w = M.w + t * M.w_nb2;
    const float r = M.res ? M.res[t * M.res_nb1 + i] : 0.0f;
    float acc = 0.0f;
    for (int s0 = 0; s0 < M.k; s0 += WS_BATCH) {
        float ev[WS_BATCH], wv[WS_BATCH];
#pragma unroll
        for (int j = 0; j < WS_BATCH; j++) {
            const int s = min(s0 + j, M.k - 1);   // clamped, unused past k
            ev[j] = e[s * M.e_nb1];
            wv[j] = w[s * M.w_nb1];
        }
        __builtin_amdgcn_sched_barrier(0);   // every load above is out before any wait
#pragma unroll
        for (int j = 0; j < WS_BATCH; j++) {
            const float p = ev[j] * wv[j];
            const float nx = s0 + j == 0 ? p : acc + p;
            acc = s0 + j < M.k ? nx : acc;
        }
    }
    if (M.res) acc = acc + r;
    M.out[t * M.out_nb1 + i] = acc;
}

void launch_moe_wsum(const moe_wsum & M, hipStream_t st) {
    launch(moe_wsum_kernel, dim3(grid1(M.n_embd, 256), (unsigned) M.n_tok), dim3(256), 0, st, M);
}

__global__ void unary_kernel(int op, float s, tview a, tview d, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const idx4 k = unflatten(i, d.ne);
    const float x = ld(at(a, k.i0, k.i1, k.i2, k.i3), a.type);
    float y;
    switch (op) {
        case 0: y = x / (1.0f + exp_cr(-x)); break;
        case 1: y = x > 0.0f ? x : 0.0f; break;
        case 2: y = 1.0f / (1.0f + exp_cr(-x)); break;
        case 3: y = x * x; break;
        case 5: y = fabsf(x); break;
        case 6: y = x > 20.0f ? x : (float) log1p(exp((double) x)); break;   // softplus, rounded once
        default: y = x * s; break;
    }
    st(at(d, k.i0, k.i1, k.i2, k.i3), d.type, y);
}

// l2_norm: one wave per row over ne0: the sum of f32 squares in double (exact for these operands
// in practice, so the order does not matter), scale = 1 / max(sqrtf(sum), eps), y = x * scale
__global__ void l2_norm_kernel(tview a, tview d, float eps, int64_t rows) {
    const int64_t r = (int64_t) blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE;
    const int lane = threadIdx.x % WAVE;
    if (r >= rows) return;
    const int64_t i1 = r % a.ne[1], i2 = (r / a.ne[1]) % a.ne[2], i3 = r / (a.ne[1] * a.ne[2]);
    double sum = 0.0;
    for (int64_t i0 = lane; i0 < a.ne[0]; i0 += WAVE) {
        const float x = ld(at(a, i0, i1, i2, i3), a.type);
        sum += (double) (x * x);
    }
    sum = wave_sum_d(sum);
    const float scale = 1.0f / fmaxf(sqrtf((float) sum), eps);
    for (int64_t i0 = lane; i0 < a.ne[0]; i0 += WAVE) st(at(d, i0, i1, i2, i3), d.type, ld(at(a, i0, i1, i2, i3), a.type) * scale);
}

void launch_l2_norm(const tview & a, const tview & dst, float eps, hipStream_t st) {
    const int64_t rows = a.ne[1] * a.ne[2] * a.ne[3];
    if (rows == 0) return;
    launch(l2_norm_kernel, dim3(grid1(rows, 4)), dim3(256), 0, st, a, dst, eps, rows);
}

// concat along dim: element i of that dim comes from a while i < a.ne[dim], else from b (same types)
__global__ void concat_kernel(tview a, tview b, tview d, int dim, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const idx4 k = unflatten(i, d.ne);
    int64_t ix[4] = { k.i0, k.i1, k.i2, k.i3 };
    const tview * s = &a;
    if (ix[dim] >= a.ne[dim]) { ix[dim] -= a.ne[dim]; s = &b; }
    const char * sp = at(*s, ix[0], ix[1], ix[2], ix[3]);
    char * dp = at(d, k.i0, k.i1, k.i2, k.i3);
    if (d.type == GGML_TYPE_F32 || d.type == GGML_TYPE_I32) *(uint32_t *) dp = *(const uint32_t *) sp;
    else *(uint16_t *) dp = *(const uint16_t *) sp;
}

void launch_concat(const tview & a, const tview & b, const tview & dst, int dim, hipStream_t st) {
    const int64_t n = nelem(dst);
    if (n == 0) return;
    launch(concat_kernel, dim3(grid1(n, 256)), dim3(256), 0, st, a, b, dst, dim, n);
}

// swiglu_split: silu(a) * b with the silu and mul ops' roundings
__global__ void glu_kernel(tview a, tview b, tview d, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const idx4 k = unflatten(i, d.ne);
    const float x = ld(at(a, k.i0, k.i1, k.i2, k.i3), a.type);
    const float g = ld(at(b, k.i0, k.i1, k.i2, k.i3), b.type);
    const float sl = x / (1.0f + exp_cr(-x));
    st(at(d, k.i0, k.i1, k.i2, k.i3), d.type, sl * g);
}

void launch_glu(const tview & a, const tview & b, const tview & dst, hipStream_t st) {
    const int64_t n = nelem(dst);
    if (n == 0) return;
    launch(glu_kernel, dim3(grid1(n, 256)), dim3(256), 0, st, a, b, dst, n);
}

// act = silu(gate) * up over 2-D f32 views (the silu and mul ops' roundings), and optionally its
// Q8_0 quantization (quantize_q8_kernel's arithmetic: a block per 32 lanes) or its Q8_K
// quantization (a workgroup's 256 elements are one super-block): one thread per element, grid.y
// over the columns
__global__ __launch_bounds__(256) void swiglu_kernel(tview g, tview u, tview d, q8_act q, q8k_act qk) {
    prefetch_kernargs<3 * sizeof(tview) + sizeof(q8_act) + sizeof(q8k_act)>();
    const int64_t K = d.ne[0], nblk = K / 32, c = blockIdx.y;
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    const bool ok = i < K;
    float v = 0.0f;
    if (ok) {
        const float x = *(const float *) at(g, i, c, 0, 0);
        const float y = x / (1.0f + exp_cr(-x));
        v = y * *(const float *) at(u, i, c, 0, 0);
        *(float *) at(d, i, c, 0, 0) = v;
    }
    if (qk.qs) {
        // K % 256 == 0: every thread holds an element
        q8k_superblock(v, threadIdx.x, qk.qs + c * K + (int64_t) blockIdx.x * 256, qk.d + c * (K / 256) + blockIdx.x,
                       qk.bsums + c * (K / 16) + (int64_t) blockIdx.x * 16);
        return;
    }
    if (!q.qs) return;
    // Q8_0 blocks of 32 consecutive elements (K % 32 == 0: a block never straddles the end)
    const float amax = group_max<32>(fabsf(v));
    const float dd = amax / 127;
    const float id = dd ? 1.0f / dd : 0.0f;
    const int qv = (int) roundf(v * id);
    const float qsum = group_sum<32>((float) qv);
    if (ok) {
        q.qs[c * K + i] = (int8_t) qv;
        if ((i % 32) == 0) {
            q.d[c * nblk + i / 32] = __half2float(__float2half_rn(dd));
            q.s[c * nblk + i / 32] = (int32_t) qsum;
        }
    }
}

void launch_swiglu(const tview & gate, const tview & up, const tview & dst, const q8_act * q, const q8k_act * qk, hipStream_t st) {
    if (dst.ne[2] != 1 || dst.ne[3] != 1 || (q && dst.ne[0] % 32) || (qk && dst.ne[0] % 256) || (q && qk)) {
        HIP_ABORT("swiglu: unsupported shape");
    }
    const q8_act none{};
    const q8k_act nonek{};
    launch(swiglu_kernel, dim3((unsigned) ((dst.ne[0] + 255) / 256), (unsigned) dst.ne[1]), dim3(256), 0, st, gate, up, dst,
           q ? *q : none, qk ? *qk : nonek);
}

void launch_unary(int op, float s, const tview & a, const tview & dst, hipStream_t st) {
    const int64_t n = nelem(dst);
    if (n == 0) return;
    launch(unary_kernel, dim3(grid1(n, 256)), dim3(256), 0, st, op, s, a, dst, n);
}

// element i (row-major over the src shape) -> element i (row-major over the dst shape)
__global__ void cpy_kernel(tview s, tview d, int64_t n) {
    prefetch_kernargs<2 * sizeof(tview) + 8>();
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const idx4 a = unflatten(i, s.ne);
    const idx4 b = unflatten(i, d.ne);
    const char * sp = at(s, a.i0, a.i1, a.i2, a.i3);
    char * dp = at(d, b.i0, b.i1, b.i2, b.i3);
    if (s.type == d.type) {
        if (s.type == GGML_TYPE_F32 || s.type == GGML_TYPE_I32) *(uint32_t *) dp = *(const uint32_t *) sp;
        else *(uint16_t *) dp = *(const uint16_t *) sp;
    } else {
        st(dp, d.type, ld(sp, s.type));
    }
}

void launch_cpy(const tview & src, const tview & dst, hipStream_t st) {
    const int64_t n = nelem(src);
    if (n == 0) return;
    launch(cpy_kernel, dim3(grid1(n, 256)), dim3(256), 0, st, src, dst, n);
}

// ---------------------------------------------------------------------------------------------
// get_rows: dst[:, i10, i11, i12] = dequant(a[:, ids[i10, i11, i12], i11, i12])

__global__ void get_rows_kernel(tview a, tview ids, tview d, const uint8_t * qs, const __half * dpl, q6k_planes q6,
                                int64_t first_block) {
    prefetch_kernargs<3 * sizeof(tview) + 16 + sizeof(q6k_planes) + 8>();
    const int64_t r = blockIdx.x;
    const int64_t i10 = r % ids.ne[0], i11 = (r / ids.ne[0]) % ids.ne[1], i12 = r / (ids.ne[0] * ids.ne[1]);
    const int32_t row = *(const int32_t *) at(ids, i10, i11, i12, 0);
    const int64_t ne00 = a.ne[0];
    float * out = (float *) at(d, 0, i10, i11, i12);
    const int64_t byte_off = row * a.nb[1] + i11 * a.nb[2] + i12 * a.nb[3];
    for (int64_t e = threadIdx.x; e < ne00; e += blockDim.x) {
        float v;
        switch (a.type) {
            case GGML_TYPE_Q4_0: {
                const int64_t blk = first_block + byte_off / 18 + e / 32;
                const int j = (int) (e % 32);
                const uint8_t b = qs[blk * Q4_0_QS + (j & 15)];
                const int q = j < 16 ? (b & 0x0F) : (b >> 4);
                v = (float) (q - 8) * __half2float(dpl[blk]);
                break;
            }
            case GGML_TYPE_Q8_0: {
                const int64_t blk = first_block + byte_off / 34 + e / 32;
                v = (float) (int8_t) qs[blk * Q8_0_QS + e % 32] * __half2float(dpl[blk]);
                break;
            }
            case GGML_TYPE_Q4_K: {
                const q4k_block * b = (const q4k_block *) (a.data + byte_off) + e / 256;
                const int k = (int) (e % 256);
                const int j = k / 32;     // sub-block
                const int l = k % 32;
                const uint8_t * s = b->scales;
                int sc, m;
                if (j < 4) { sc = s[j] & 63; m = s[j + 4] & 63; }
                else { sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4); m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4); }
                const uint8_t qb = b->qs[32 * (j / 2) + l];
                const int q = (j & 1) ? (qb >> 4) : (qb & 0x0F);
                const float dd = __half2float(b->d) * (float) sc;
                const float mm = __half2float(b->dmin) * (float) m;
                v = dd * (float) q - mm;
                break;
            }
            case GGML_TYPE_Q5_K: {
                const q5k_block * b = (const q5k_block *) (a.data + byte_off) + e / 256;
                const int k = (int) (e % 256);
                const int j = k / 32, l = k % 32;
                const uint8_t * s = b->scales;
                int sc, m;
                if (j < 4) { sc = s[j] & 63; m = s[j + 4] & 63; }
                else { sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4); m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4); }
                const uint8_t qb = b->qs[32 * (j / 2) + l];
                const int q = ((j & 1) ? (qb >> 4) : (qb & 0x0F)) + 16 * ((b->qh[l] >> j) & 1);
                const float dd = __half2float(b->d) * (float) sc;
                const float mm = __half2float(b->dmin) * (float) m;
                v = dd * (float) q - mm;
                break;
            }
            case GGML_TYPE_Q6_K: {
                const int64_t blk = first_block + byte_off / 210 + e / 256;
                const int k = (int) (e % 256);
                const int h = k / 128, g = (k % 128) / 32, l = k % 32;
                const int lo = (q6.ql[blk * 128 + 64 * h + 32 * (g & 1) + l] >> (4 * (g >> 1))) & 0x0F;
                const int hi = (q6.qh[blk * 64 + 32 * h + l] >> (2 * g)) & 3;
                const float ds = __half2float(q6.d[blk]) * (float) q6.sc[blk * 16 + 8 * h + 2 * g + l / 16];
                v = ds * (float) ((lo | (hi << 4)) - 32);
                break;
            }
            default:
                v = ld(a.data + byte_off + e * a.nb[0], a.type);
                break;
        }
        out[e] = v;
    }
}

void launch_get_rows(const tview & a, const tview & ids, const tview & dst, const uint8_t * qs_plane,
                     const __half * d_plane, const q6k_planes & q6, int64_t first_block, hipStream_t st) {
    const int64_t rows = ids.ne[0] * ids.ne[1] * ids.ne[2];
    if (rows == 0) return;
    launch(get_rows_kernel, dim3((unsigned) rows), dim3(256), 0, st, a, ids, dst, qs_plane, d_plane, q6, first_block);
}

// ---------------------------------------------------------------------------------------------
// RoPE: one thread per rotated pair of one (head, token) row

// pair li of a RoPE job (row-major over pairs of the src rows); the result is stored in dst's type.
// IDX: the index type of the unflattening (32-bit when the job's items fit, which costs a fraction
// of the 64-bit divisions: this kernel's time is mostly its index arithmetic)
template <typename IDX>
__device__ __forceinline__ void rope_pair(const rope_job & J, IDX li) {
    const tview & x = J.src;
    const tview & d = J.dst;
    const rope_params & p = J.p;
    const IDX half = (IDX) (x.ne[0] / 2), n1 = (IDX) x.ne[1], n2 = (IDX) x.ne[2];
    const IDX ip = li % half;
    IDX r = li / half;
    const IDX i1 = r % n1; r /= n1;
    const IDX i2 = r % n2; r /= n2;
    const IDX i3 = r;
    const int i0 = (int) (2 * ip);
    if (i0 >= p.n_dims) {
        for (int k = 0; k < 2; k++) st(at(d, i0 + k, i1, i2, i3), d.type, *(const float *) at(x, i0 + k, i1, i2, i3));
        return;
    }
    float c, sn;
    if (J.cs) {
        const float2 v = J.cs[i2 * (p.n_dims / 2) + i0 / 2];
        c = v.x;
        sn = v.y;
    } else {
        rope_pair_cs(p, J.ff, J.pos[i2], i0 / 2, c, sn);
    }
    int64_t a0, a1;
    if (p.mode & GGML_ROPE_TYPE_NEOX) { a0 = i0 / 2; a1 = i0 / 2 + p.n_dims / 2; }
    else { a0 = i0; a1 = i0 + 1; }
    const float x0 = *(const float *) at(x, a0, i1, i2, i3);
    const float x1 = *(const float *) at(x, a1, i1, i2, i3);
    st(at(d, a0, i1, i2, i3), d.type, x0 * c - x1 * sn);
    st(at(d, a1, i1, i2, i3), d.type, x0 * sn + x1 * c);
}

// element li of a copy job (row-major over src, written row-major over dst, converted to dst's type)
template <typename IDX>
__device__ __forceinline__ void copy_elem(const rope_job & J, IDX li) {
    auto unflat = [](IDX i, const int64_t ne[4], IDX (&o)[4]) {
        const IDX n0 = (IDX) ne[0], n1 = (IDX) ne[1], n2 = (IDX) ne[2];
        o[0] = i % n0; i /= n0;
        o[1] = i % n1; i /= n1;
        o[2] = i % n2; o[3] = i / n2;
    };
    IDX a[4], b[4];
    unflat(li, J.src.ne, a);
    const bool same = J.src.ne[0] == J.dst.ne[0] && J.src.ne[1] == J.dst.ne[1] && J.src.ne[2] == J.dst.ne[2];
    if (same) { b[0] = a[0]; b[1] = a[1]; b[2] = a[2]; b[3] = a[3]; }
    else unflat(li, J.dst.ne, b);
    st(at(J.dst, b[0], b[1], b[2], b[3]), J.dst.type, ld(at(J.src, a[0], a[1], a[2], a[3]), J.src.type));
}

// Row r of a RoPE job with a QK-Norm, by one wave: the row's sum of squares in double and
// scale = 1 / sqrtf((float) (sum / hd) + eps), as the rms_norm op forms them; y = (x * scale) * w
// (the norm's mul) into the wave's LDS row; then each rotation pair as rope_pair rotates it.
constexpr int ROPE_NORM_MAX_HD = 256;
__device__ __forceinline__ void rope_norm_row(const rope_job & J, int64_t r, int lane, float * s_row) {
    const int hd = (int) J.src.ne[0];
    const int64_t i1 = r % J.src.ne[1], i2 = r / J.src.ne[1];   // (head, token); ne[3] == 1
    const float * xr = J.norm_x + i1 * J.norm_nb1 + i2 * J.norm_nb2;
    constexpr int PER = ROPE_NORM_MAX_HD / WAVE;
    float xv[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) xv[k] = xr[min(lane + WAVE * k, hd - 1)];   // clamped, unused past hd
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < PER; k++) if (lane + WAVE * k < hd) ss += (double) (xv[k] * xv[k]);
    ss = wave_sum_d(ss);
    const float scale = 1.0f / sqrtf((float) (ss / (double) hd) + J.norm_eps);
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int e = lane + WAVE * k;
        if (e < hd) s_row[e] = (xv[k] * scale) * J.norm_w[e];
    }
    // the wave's LDS writes are visible to its own later reads (in order within a wave)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const rope_params & p = J.p;
    const int half = p.n_dims / 2;
    const bool neox = (p.mode & GGML_ROPE_TYPE_NEOX) != 0;
    for (int ip = lane; ip < half; ip += WAVE) {
        float c, sn;
        if (J.cs) {
            const float2 v = J.cs[i2 * half + ip];
            c = v.x;
            sn = v.y;
        } else {
            rope_pair_cs(p, J.ff, J.pos[i2], ip, c, sn);
        }
        const int a0 = neox ? ip : 2 * ip, a1 = neox ? ip + half : 2 * ip + 1;
        const float x0 = s_row[a0], x1 = s_row[a1];
        st(at(J.dst, a0, i1, i2, 0), J.dst.type, x0 * c - x1 * sn);
        st(at(J.dst, a1, i1, i2, 0), J.dst.type, x0 * sn + x1 * c);
    }
    for (int e = p.n_dims + lane; e < hd; e += WAVE) st(at(J.dst, e, i1, i2, 0), J.dst.type, s_row[e]);
}

// Independent RoPE and copy jobs of one decode step in one launch (Q rotation; K rotation stored
// straight into the F16 KV cache; V appended to it). Each job owns a whole number of workgroups.
__global__ __launch_bounds__(256) void rope_batch_kernel(const rope_batch B) {
    prefetch_kernargs<sizeof(rope_batch)>();
    __shared__ float s_rows[256 / WAVE][ROPE_NORM_MAX_HD];
    int j = 0;
#pragma unroll
    for (int k = 1; k < ROPE_MAX_JOBS; k++) if (k < B.n_jobs && (int64_t) blockIdx.x >= B.first_block[k]) j = k;
    const rope_job & J = B.job[j];
    if (J.norm_x) {
        // one wave per row (no workgroup barrier: a wave past the rows just ends)
        const int wave = threadIdx.x / WAVE;
        const int64_t r = ((int64_t) blockIdx.x - B.first_block[j]) * (256 / WAVE) + wave;
        if (r < J.n) rope_norm_row(J, r, threadIdx.x % WAVE, s_rows[wave]);
        return;
    }
    const int64_t li = ((int64_t) blockIdx.x - B.first_block[j]) * blockDim.x + threadIdx.x;
    if (li >= J.n) return;
    if (J.n <= (int64_t) UINT32_MAX) {
        if (J.pos) rope_pair<uint32_t>(J, (uint32_t) li);
        else copy_elem<uint32_t>(J, (uint32_t) li);
    } else {
        if (J.pos) rope_pair<int64_t>(J, li);
        else copy_elem<int64_t>(J, li);
    }
}

void launch_rope_batch(rope_batch & B, hipStream_t st) {
    int64_t blocks = 0;
    for (int k = 0; k < B.n_jobs; k++) {
        const rope_job & J = B.job[k];
        if (J.norm_x && (J.src.ne[0] > ROPE_NORM_MAX_HD || J.src.ne[3] != 1 || J.n != J.src.ne[1] * J.src.ne[2] || !J.pos ||
                         J.p.n_dims > J.src.ne[0])) {
            HIP_ABORT("rope: a QK-Norm job needs rows of at most %d floats", ROPE_NORM_MAX_HD);
        }
        B.first_block[k] = blocks;
        blocks += J.norm_x ? grid1(J.n, 256 / WAVE) : grid1(J.n, 256);
    }
    if (blocks == 0) return;
    launch(rope_batch_kernel, dim3((unsigned) blocks), dim3(256), 0, st, B);
}

// one thread per (token, rotation pair): rope_pair_cs (theta after ip multiplications by
// theta_scale in float, as the CPU cache builds it; then the correctly rounded cos and sin)
__global__ void rope_table_kernel(const int32_t * pos, int64_t n_pos, rope_params p, const float * ff, float2 * out) {
    const int half = p.n_dims / 2;
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_pos * half) return;
    float c, s;
    rope_pair_cs(p, ff, pos[i / half], (int) (i % half), c, s);
    out[i] = make_float2(c, s);
}

void launch_rope_table(const int32_t * pos, int64_t n_pos, const rope_params & p, const float * ff, float2 * out, hipStream_t st) {
    const int64_t n = n_pos * (p.n_dims / 2);
    if (n <= 0) return;
    launch(rope_table_kernel, dim3(grid1(n, 256)), dim3(256), 0, st, pos, n_pos, p, ff, out);
}

void launch_rope(const tview & src, const int32_t * pos, const float * freq_factors, const tview & dst,
                 const rope_params & p, hipStream_t st) {
    rope_batch B{};
    B.n_jobs = 1;
    B.job[0] = rope_job{ src, dst, pos, freq_factors, p, nelem(src) / 2 };
    launch_rope_batch(B, st);
}

// ---------------------------------------------------------------------------------------------
// softmax over ne0 of each row: y = exp(w - max) / sum, w = x*scale + slope*mask

__global__ __launch_bounds__(256) void soft_max_kernel(tview a, tview m, int has_mask, tview d, float scale,
                                                        float m0, float m1, uint32_t n_head_log2, float max_bias) {
    __shared__ float s_red[4];
    __shared__ double s_sum[4];
    const int64_t r = blockIdx.x;
    const int64_t i1 = r % a.ne[1], i2 = (r / a.ne[1]) % a.ne[2], i3 = r / (a.ne[1] * a.ne[2]);
    const int t = threadIdx.x;
    const int64_t nc = a.ne[0];
    float slope = 1.0f;
    if (max_bias > 0.0f) {
        const uint32_t h = (uint32_t) i2;
        slope = h < n_head_log2 ? powf(m0, (float) (h + 1)) : powf(m1, (float) (2 * (h - n_head_log2) + 1));
    }
    float mx = -INFINITY;
    for (int64_t i = t; i < nc; i += 256) {
        float w = *(const float *) at(a, i, i1, i2, i3) * scale;
        if (has_mask) w += slope * ld(at(m, i, i1, i2 % m.ne[2], i3 % m.ne[3]), m.type);
        *(float *) at(d, i, i1, i2, i3) = w;
        mx = fmaxf(mx, w);
    }
    mx = wave_max(mx);
    if ((t % 64) == 0) s_red[t / 64] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    double sum = 0.0;
    for (int64_t i = t; i < nc; i += 256) {
        float * p = (float *) at(d, i, i1, i2, i3);
        const float v = exp_cr(*p - mx);
        *p = v;
        sum += (double) v;
    }
    sum = wave_sum_d(sum);
    if ((t % 64) == 0) s_sum[t / 64] = sum;
    __syncthreads();
    const double total = s_sum[0] + s_sum[1] + s_sum[2] + s_sum[3];
    const float inv = (float) (1.0 / total);
    for (int64_t i = t; i < nc; i += 256) *(float *) at(d, i, i1, i2, i3) *= inv;
}

void launch_soft_max(const tview & a, const tview * mask, const tview & dst, float scale, float max_bias, hipStream_t st) {
    const int64_t rows = a.ne[1] * a.ne[2] * a.ne[3];
    const uint32_t n_head = (uint32_t) a.ne[2];
    const uint32_t n_head_log2 = n_head ? 1u << (uint32_t) floor(log2((double) n_head)) : 1u;
    const float m0 = powf(2.0f, -(max_bias) / n_head_log2);
    const float m1 = powf(2.0f, -(max_bias / 2.0f) / n_head_log2);
    tview m{};
    if (mask) m = *mask;
    launch(soft_max_kernel, dim3((unsigned) rows), dim3(256), 0, st, a, m, mask ? 1 : 0, dst, scale, m0, m1, n_head_log2, max_bias);
}

// ---------------------------------------------------------------------------------------------
// MoE routing (one workgroup per token)

__global__ __launch_bounds__(256) void moe_route_kernel(const moe_route R) {
    prefetch_kernargs<sizeof(moe_route)>();
    __shared__ float s_p[MOE_ROUTE_MAX_EXPERTS];
    __shared__ int s_ids[MOE_ROUTE_MAX_K];
    __shared__ int s_cnt[256];
    __shared__ __align__(16) uint64_t s_key[256];   // read as 16-byte pairs
    __shared__ float s_red[4];
    __shared__ double s_sum[4];
    const int t = threadIdx.x, tok = blockIdx.x, E = R.n_expert;
    const float * lg = R.logits + (int64_t) tok * R.logits_nb1;
    if (E <= 256) {
        // the routing the expert GEMV of a one-token step runs in its own workgroups
        moe_route_256(t < E ? lg[t] * R.scale : -INFINITY, E, R.k, s_p, s_ids, s_cnt, s_key, s_red, s_sum);
    } else {
        if (t < R.k) s_ids[t] = 0;   // (every slot is written below unless a probability is NaN)
        // softmax, as soft_max_kernel
        float mx = -INFINITY;
        for (int i = t; i < E; i += 256) {
            const float w = lg[i] * R.scale;
            s_p[i] = w;
            mx = fmaxf(mx, w);
        }
        mx = wave_max(mx);
        if ((t % 64) == 0) s_red[t / 64] = mx;
        __syncthreads();
        mx = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
        double sum = 0.0;
        for (int i = t; i < E; i += 256) {
            const float v = exp_cr(s_p[i] - mx);
            s_p[i] = v;
            sum += (double) v;
        }
        sum = wave_sum_d(sum);
        if ((t % 64) == 0) s_sum[t / 64] = sum;
        __syncthreads();
        const float inv = (float) (1.0 / (s_sum[0] + s_sum[1] + s_sum[2] + s_sum[3]));
        for (int i = t; i < E; i += 256) s_p[i] *= inv;
        __syncthreads();
        // position of each expert in the stable descending order; the first k positions are the top-k
        for (int i = t; i < E; i += 256) {
            const float v = s_p[i];
            int rank = 0;
            for (int j = 0; j < E; j++) {
                const float u = s_p[j];
                rank += (u > v || (u == v && j < i)) ? 1 : 0;
            }
            if (rank < R.k) s_ids[rank] = i;
        }
        __syncthreads();
    }
    if (t == 0) moe_route_store(s_p, s_ids, R.k, R.ids + (int64_t) tok * R.ids_nb1, R.w + (int64_t) tok * R.w_nb1);
}

void launch_moe_route(const moe_route & R, hipStream_t st) {
    if (R.n_expert < 1 || R.n_expert > MOE_ROUTE_MAX_EXPERTS || R.k < 1 || R.k > MOE_ROUTE_MAX_K || R.k > R.n_expert) {
        HIP_ABORT("moe_route: %d experts, k=%d unsupported", R.n_expert, R.k);
    }
    if (R.n_tok < 1) return;
    launch(moe_route_kernel, dim3((unsigned) R.n_tok), dim3(256), 0, st, R);
}

// ---------------------------------------------------------------------------------------------
// argmax of each row (first index of the maximum)

__global__ __launch_bounds__(256) void argmax_kernel(tview a, int32_t * out) {
    __shared__ float s_v[4];
    __shared__ int s_i[4];
    const int64_t r = blockIdx.x;
    const int t = threadIdx.x;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int64_t i = t; i < a.ne[0]; i += 256) {
        const float v = *(const float *) at(a, i, r, 0, 0);
        if (v > bv) { bv = v; bi = (int) i; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float v2 = __shfl_xor(bv, o, WAVE);
        const int i2 = __shfl_xor(bi, o, WAVE);
        if (v2 > bv || (v2 == bv && i2 < bi)) { bv = v2; bi = i2; }
    }
    if ((t % 64) == 0) { s_v[t / 64] = bv; s_i[t / 64] = bi; }
    __syncthreads();
    if (t == 0) {
        for (int w = 1; w < 4; w++) if (s_v[w] > bv || (s_v[w] == bv && s_i[w] < bi)) { bv = s_v[w]; bi = s_i[w]; }
        if (bi == 0x7fffffff) bi = 0;
        out[r] = bi;
    }
}

// One wide row (the logits of the greedy pick): ARGMAX_PARTS workgroups reduce consecutive chunks
// to (value, first index), then one workgroup reduces the parts in order of their indices. The
// comparisons are the one-pass rule's (strictly greater wins, so the first index of the maximum;
// nothing above -inf: index 0).
__device__ __forceinline__ void argmax_merge(float & bv, int & bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

__device__ void argmax_block(float & bv, int & bi) {
    __shared__ float s_v[4];
    __shared__ int s_i[4];
    const int t = threadIdx.x;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) argmax_merge(bv, bi, __shfl_xor(bv, o, WAVE), __shfl_xor(bi, o, WAVE));
    if ((t % 64) == 0) { s_v[t / 64] = bv; s_i[t / 64] = bi; }
    __syncthreads();
    bv = s_v[0];
    bi = s_i[0];
    for (int w = 1; w < 4; w++) argmax_merge(bv, bi, s_v[w], s_i[w]);
}

__global__ __launch_bounds__(256) void argmax_parts_kernel(tview a, int64_t chunk, float * pv, int * pi) {
    prefetch_kernargs<sizeof(tview) + 24>();
    const int64_t i0 = (int64_t) blockIdx.x * chunk, i1 = min(i0 + chunk, a.ne[0]);
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int64_t i = i0 + threadIdx.x; i < i1; i += 256) {
        const float v = *(const float *) at(a, i, 0, 0, 0);
        if (v > bv) { bv = v; bi = (int) i; }
    }
    argmax_block(bv, bi);
    if (threadIdx.x == 0) { pv[blockIdx.x] = bv; pi[blockIdx.x] = bi; }
}

__global__ __launch_bounds__(256) void argmax_final_kernel(const float * pv, const int * pi, int n_parts, int32_t * out,
                                                           int32_t * out2, int32_t * out3) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    if ((int) threadIdx.x < n_parts) { bv = pv[threadIdx.x]; bi = pi[threadIdx.x]; }
    argmax_block(bv, bi);
    if (threadIdx.x == 0) {
        const int32_t r = bi == 0x7fffffff ? 0 : bi;
        out[0] = r;
        if (out2) out2[0] = r;
        if (out3) out3[0] = r;
    }
}

void launch_argmax(const tview & a, int32_t * out, hipStream_t st) {
    launch(argmax_kernel, dim3((unsigned) a.ne[1]), dim3(256), 0, st, a, out);
}

void launch_argmax_row(const tview & a, int32_t * out, float * part_v, int * part_i, hipStream_t st, int32_t * out2,
                       int32_t * out3) {
    if (a.ne[1] != 1 || a.ne[2] != 1 || a.ne[3] != 1 || a.ne[0] <= 0 || a.ne[0] > INT32_MAX) HIP_ABORT("argmax_row: one row expected");
    const int64_t chunk = (a.ne[0] + ARGMAX_PARTS - 1) / ARGMAX_PARTS;
    const int parts = (int) ((a.ne[0] + chunk - 1) / chunk);
    launch(argmax_parts_kernel, dim3((unsigned) parts), dim3(256), 0, st, a, chunk, part_v, part_i);
    launch(argmax_final_kernel, dim3(1), dim3(256), 0, st, (const float *) part_v, (const int *) part_i, parts, out, out2, out3);
}

// ---------------------------------------------------------------------------------------------
// generic mul_mat (F32/F16/BF16 src0, rows contiguous): one wave per output element.
// src1 is first rounded to src0's type, as ggml converts it to the weight's dot type.

__global__ __launch_bounds__(256) void mul_mat_generic_kernel(tview s0, tview s1, tview d, int64_t n_out) {
    const int64_t o = (int64_t) blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE;
    if (o >= n_out) return;
    const int lane = threadIdx.x % WAVE;
    const idx4 k = unflatten(o, d.ne);    // (i01, i11, i12, i13)
    const int64_t r2 = s1.ne[2] / s0.ne[2], r3 = s1.ne[3] / s0.ne[3];
    const char * a = at(s0, 0, k.i0, k.i2 / r2, k.i3 / r3);
    const int64_t K = s0.ne[0];
    // products rounded to float, summed in double, as ggml-cpu's f16/f32 vec_dot
    double acc = 0.0;
    for (int64_t i = lane; i < K; i += WAVE) {
        const float w = ld(a + i * s0.nb[0], s0.type);
        float x = *(const float *) at(s1, i, k.i1, k.i2, k.i3);
        if (s0.type == GGML_TYPE_F16) x = __half2float(__float2half_rn(x));
        else if (s0.type == GGML_TYPE_BF16) {
            uint32_t u = __float_as_uint(x);
            u = (u + (0x7fffu + ((u >> 16) & 1u))) & 0xffff0000u;
            x = __uint_as_float(u);
        }
        acc += (double) (w * x);
    }
    acc = wave_sum_d(acc);
    if (lane == 0) *(float *) at(d, k.i0, k.i1, k.i2, k.i3) = (float) acc;
}

// F32 / F16 weights with contiguous 16-byte aligned rows (the MoE router, F16 score products): one
// wave per output, each lane reading 8 consecutive elements of the row and of the activation per
// chunk, MR_BATCH chunks of loads in flight before the first product; same float products summed
// in double as above.
constexpr int MR_BATCH = 4;

template <int TYPE>
__global__ __launch_bounds__(256) void mul_mat_rows_kernel(tview s0, tview s1, tview d, int64_t n_out) {
    const int64_t o = (int64_t) blockIdx.x * (blockDim.x / WAVE) + threadIdx.x / WAVE;
    if (o >= n_out) return;
    const int lane = threadIdx.x % WAVE;
    const idx4 k = unflatten(o, d.ne);
    const int64_t r2 = s1.ne[2] / s0.ne[2], r3 = s1.ne[3] / s0.ne[3];
    const char * a = at(s0, 0, k.i0, k.i2 / r2, k.i3 / r3);
    const float * x = (const float *) at(s1, 0, k.i1, k.i2, k.i3);
    const int nch = (int) (s0.ne[0] / 8);
    double acc = 0.0;
    for (int c0 = 0; c0 < nch; c0 += MR_BATCH * WAVE) {
        float w[MR_BATCH][8], v[MR_BATCH][8];
#pragma unroll
        for (int j = 0; j < MR_BATCH; j++) {
            const int c = min(c0 + j * WAVE + lane, nch - 1);
            const float4 x0 = ((const float4 *) x)[2 * c], x1 = ((const float4 *) x)[2 * c + 1];
            v[j][0] = x0.x; v[j][1] = x0.y; v[j][2] = x0.z; v[j][3] = x0.w;
            v[j][4] = x1.x; v[j][5] = x1.y; v[j][6] = x1.z; v[j][7] = x1.w;
            if (TYPE == GGML_TYPE_F32) {
                const float4 a0 = ((const float4 *) a)[2 * c], a1 = ((const float4 *) a)[2 * c + 1];
                w[j][0] = a0.x; w[j][1] = a0.y; w[j][2] = a0.z; w[j][3] = a0.w;
                w[j][4] = a1.x; w[j][5] = a1.y; w[j][6] = a1.z; w[j][7] = a1.w;
            } else {
                const uint4 h = ((const uint4 *) a)[c];
                const uint32_t hw[4] = { h.x, h.y, h.z, h.w };
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float2 f = __half22float2(*(const __half2 *) &hw[e]);
                    w[j][2 * e] = f.x; w[j][2 * e + 1] = f.y;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < MR_BATCH; j++) {
            if (c0 + j * WAVE + lane >= nch) continue;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float xv = TYPE == GGML_TYPE_F16 ? __half2float(__float2half_rn(v[j][e])) : v[j][e];
                acc += (double) (w[j][e] * xv);
            }
        }
    }
    acc = wave_sum_d(acc);
    if (lane == 0) *(float *) at(d, k.i0, k.i1, k.i2, k.i3) = (float) acc;
}

// The MoE router with the FFN norm folded in: y = rms_norm(x) * nw computed by every workgroup of
// a column into LDS (the rms_norm_kernel's partition and roundings: per-thread double sums of
// squares over i = t, t + 256, ..., the four wave sums in order, mean and scale in float, then
// (x * scale) * nw), written to y_out by the column's first workgroup for the other consumers, and
// the F32 router rows dotted with it as mul_mat_rows_kernel does (same lane partition, float
// products summed in double). One wave per router row, 4 rows per workgroup, grid.y = columns.
__global__ __launch_bounds__(256) void mul_mat_rows_norm_kernel(tview w, const float * __restrict__ x, int64_t x_stride,
                                                                const float * __restrict__ nw, float eps,
                                                                float * __restrict__ y_out, int64_t y_stride, tview d,
                                                                q8k_act q8k) {
    prefetch_kernargs<2 * sizeof(tview) + 48 + sizeof(q8k_act)>();
    extern __shared__ __align__(16) float s_y[];      // [K]
    __shared__ double s_part[4];
    const int64_t K = w.ne[0], col = blockIdx.y;
    const int t = threadIdx.x, lane = t % WAVE, wave = t / WAVE;
    const float * xc = x + col * x_stride;
    const int64_t o = (int64_t) blockIdx.x * 4 + wave;   // this wave's output row
    const float * a = (const float *) (w.data + min(o, w.ne[1] - 1) * w.nb[1]);   // clamped; not stored past the end
    const int nch = (int) (K / 8);
    // Loads first, none depending on another and in the order they are used (loads complete in
    // issue order): the column, the norm weight, then the first batch of this wave's weight row
    // (which does not depend on the column). Up to RB * 256 elements (the MoE router's 2048) they
    // are one straight batch: a loop of load -> use puts one round trip per iteration on the path,
    // and a loop header makes the compiler wait for every load in flight. Indices clamped, values
    // past the ends unused.
    constexpr int RB = 8;
    const bool one_batch = K <= RB * 256;
    float xv[RB], nv[RB];
    if (one_batch) {
#pragma unroll
        for (int j = 0; j < RB; j++) xv[j] = xc[min((int64_t) t + j * 256, K - 1)];
#pragma unroll
        for (int j = 0; j < RB; j++) nv[j] = nw[min((int64_t) t + j * 256, K - 1)];
    }
    float4 wa[MR_BATCH][2];
#pragma unroll
    for (int j = 0; j < MR_BATCH; j++) {
        const int c = min(j * WAVE + lane, nch - 1);
        wa[j][0] = ((const float4 *) a)[2 * c];
        wa[j][1] = ((const float4 *) a)[2 * c + 1];
    }
    double sum = 0.0;
    if (one_batch) {
#pragma unroll
        for (int j = 0; j < RB; j++) {
            const int64_t i = t + j * 256;
            if (i < K) {
                s_y[i] = xv[j];
                sum += (double) (xv[j] * xv[j]);
            }
        }
    } else {
        for (int64_t i = t; i < K; i += 256) {
            const float v = xc[i];
            s_y[i] = v;
            sum += (double) (v * v);
        }
    }
    sum = wave_sum_d(sum);
    if (lane == 0) s_part[wave] = sum;
    __syncthreads();
    const double total = s_part[0] + s_part[1] + s_part[2] + s_part[3];
    const float mean = (float) (total / (double) K);
    const float scale = 1.0f / sqrtf(mean + eps);
    if (one_batch) {
#pragma unroll
        for (int j = 0; j < RB; j++) {
            const int64_t i = t + j * 256;
            if (i < K) {
                const float on = (s_y[i] * scale) * nv[j];
                s_y[i] = on;
                if (blockIdx.x == 0) y_out[col * y_stride + i] = on;
            }
        }
    } else {
        for (int64_t i = t; i < K; i += 256) {
            const float on = (s_y[i] * scale) * nw[i];
            s_y[i] = on;
            if (blockIdx.x == 0) y_out[col * y_stride + i] = on;
        }
    }
    __syncthreads();
    // the normalized column's Q8_K form for the norm's quantized consumers (q8k set): workgroup x
    // quantizes super-blocks x, x + gridDim.x, ... (every workgroup holds the whole column)
    if (q8k.qs) {
        const int64_t nsb = K / 256;
        for (int64_t sb = blockIdx.x; sb < nsb; sb += gridDim.x) {
            q8k_superblock(s_y[sb * 256 + t], t, q8k.qs + col * K + sb * 256, q8k.d + col * nsb + sb,
                           q8k.bsums + col * (K / 16) + sb * 16);
        }
    }
    if (o >= w.ne[1]) return;
    double acc = 0.0;
    for (int c0 = 0; c0 < nch; c0 += MR_BATCH * WAVE) {
        // the first batch's weights are already in registers; later batches load here
        if (c0 > 0) {
#pragma unroll
            for (int j = 0; j < MR_BATCH; j++) {
                const int c = min(c0 + j * WAVE + lane, nch - 1);
                wa[j][0] = ((const float4 *) a)[2 * c];
                wa[j][1] = ((const float4 *) a)[2 * c + 1];
            }
        }
        float wv[MR_BATCH][8], v[MR_BATCH][8];
#pragma unroll
        for (int j = 0; j < MR_BATCH; j++) {
            const int c = min(c0 + j * WAVE + lane, nch - 1);
            const float4 x0 = ((const float4 *) s_y)[2 * c], x1 = ((const float4 *) s_y)[2 * c + 1];
            v[j][0] = x0.x; v[j][1] = x0.y; v[j][2] = x0.z; v[j][3] = x0.w;
            v[j][4] = x1.x; v[j][5] = x1.y; v[j][6] = x1.z; v[j][7] = x1.w;
            wv[j][0] = wa[j][0].x; wv[j][1] = wa[j][0].y; wv[j][2] = wa[j][0].z; wv[j][3] = wa[j][0].w;
            wv[j][4] = wa[j][1].x; wv[j][5] = wa[j][1].y; wv[j][6] = wa[j][1].z; wv[j][7] = wa[j][1].w;
        }
#pragma unroll
        for (int j = 0; j < MR_BATCH; j++) {
            if (c0 + j * WAVE + lane >= nch) continue;
#pragma unroll
            for (int e = 0; e < 8; e++) acc += (double) (wv[j][e] * v[j][e]);
        }
    }
    acc = wave_sum_d(acc);
    if (lane == 0) *(float *) at(d, o, col, 0, 0) = (float) acc;
}

bool mul_mat_rows_norm_supported(const tview & w, int64_t K) {
    return w.type == GGML_TYPE_F32 && w.ne[0] == K && K % 8 == 0 && K <= MUL_MAT_ROWS_NORM_MAX_K && w.nb[0] == 4 &&
           w.ne[2] == 1 && w.ne[3] == 1 && ((uintptr_t) w.data % 16) == 0 && w.nb[1] % 16 == 0;
}

void launch_mul_mat_rows_norm(const tview & w, const float * x, int64_t x_stride, const float * nw, float eps, float * y_out,
                              int64_t y_stride, const tview & dst, int64_t ncols, q8k_act q8k, hipStream_t st) {
    if (!mul_mat_rows_norm_supported(w, w.ne[0]) || dst.ne[0] != w.ne[1] || dst.ne[1] != ncols || dst.nb[0] != 4 ||
        (q8k.qs && w.ne[0] % 256)) {
        HIP_ABORT("mul_mat_rows_norm: unsupported operands");
    }
    launch(mul_mat_rows_norm_kernel, dim3((unsigned) ((w.ne[1] + 3) / 4), (unsigned) ncols), dim3(256),
           (size_t) w.ne[0] * sizeof(float), st, w, x, x_stride, nw, eps, y_out, y_stride, dst, q8k);
}

void launch_mul_mat_generic(const tview & src0, const tview & src1, const tview & dst, hipStream_t st) {
    const int64_t n = nelem(dst);
    if (n == 0) return;
    const int64_t es = src0.type == GGML_TYPE_F32 ? 4 : 2;
    const bool rows = (src0.type == GGML_TYPE_F32 || src0.type == GGML_TYPE_F16) && src0.ne[0] % 8 == 0 &&
                      src0.nb[0] == es && src1.nb[0] == 4 && ((uintptr_t) src0.data | (uintptr_t) src1.data) % 16 == 0 &&
                      src0.nb[1] % 16 == 0 && src0.nb[2] % 16 == 0 && src0.nb[3] % 16 == 0 &&
                      src1.nb[1] % 16 == 0 && src1.nb[2] % 16 == 0 && src1.nb[3] % 16 == 0;
    if (rows && src0.type == GGML_TYPE_F32) launch(mul_mat_rows_kernel<GGML_TYPE_F32>, dim3(grid1(n, 4)), dim3(256), 0, st, src0, src1, dst, n);
    else if (rows) launch(mul_mat_rows_kernel<GGML_TYPE_F16>, dim3(grid1(n, 4)), dim3(256), 0, st, src0, src1, dst, n);
    else launch(mul_mat_generic_kernel, dim3(grid1(n, 4)), dim3(256), 0, st, src0, src1, dst, n);
}
