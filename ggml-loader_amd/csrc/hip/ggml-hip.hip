// ggml-hip.hip — the gfx950 ggml backend: device buffers, host<->device tensor transfers (with
// the weight-plane repack of Q4_0/Q8_0), and graph execution.
//
// graph_compute walks the ggml graph in node order (the order ggml-cpu executes, which the
// reference relies on for the KV-cache writes: model.cpp:1413-1414 precede the attention reads)
// and issues kernels on the backend's stream. With fusion on (default), it recognizes the
// per-token patterns of build_graph (reference model.cpp:1296-1474) and runs them as fused
// kernels:
//   rms_norm -> mul(weight)                 one kernel, also emitting the Q8_0/Q8_K activation
//   mul_mat x {q,k,v} sharing one input     one multi-matrix GEMV launch
//   mul_mat(gate), mul_mat(up), silu, mul   one GEMV launch with a SwiGLU epilogue (+ Q8_0 act)
//   mul_mat -> add(residual)                the residual add in the GEMV epilogue
//   K^T Q -> soft_max -> cont(V^T) -> V KQ -> permute -> cont
//                                           split-KV decode attention (+ Q8_0 act of its output)
// Everything else runs one kernel per node. Intermediate tensors swallowed by a fusion are not
// written (they have no other consumer and are not graph outputs). The graph allocator does not
// recycle memory inside a graph for this backend's buffers (buffer type flag), so executing a
// fused group at its first member's position can never clobber a live tensor.
#include "ggml-hip.h"
#include "ggml-backend-impl.h"
#include "kernels.h"

#include <algorithm>
#include <chrono>
#include <climits>
#include <cmath>
#include <cstring>
#include <map>
#include <string>
#include <unordered_map>
#include <vector>

thread_local launch_timing g_launch_timing;

namespace {

// ---------------------------------------------------------------------------------------------
// devices

// Scratch of ggml_backend_hip_graph_compute_static: the kernels' partial results (attention
// scores and partials, quantized activations, expert groups, argmax parts) for callers that cannot
// allocate. Every GPU the library runs on holds its own copy until the process ends; host code
// uses the per-device address hipGetSymbolAddress resolves (hip_device::static_scratch), never
// this name.
static __device__ __align__(256) uint8_t scratch[GGML_HIP_STATIC_SCRATCH_BYTES];

struct hip_device {
    int id = 0;
    bool ready = false;
    hipStream_t stream = nullptr;
    // this device's copy of `scratch` (nullptr until resolved at backend init)
    uint8_t * static_scratch = nullptr;
    // device staging for repacked uploads/downloads
    uint8_t * staging = nullptr;
    size_t staging_size = 0;
    // pinned host ring for small uploads: tensor_set copies the bytes into it and queues the copy
    // on the stream without waiting; the ring starts over whenever the stream has drained
    uint8_t * up_ring = nullptr;
    size_t up_off = 0;
    // pinned host landing area for downloads
    uint8_t * down = nullptr;
    size_t down_size = 0;
    // token sampling: device words (3 result ints, then the penalty table) and the sorted path's
    // workspace
    int * smp = nullptr;
    size_t smp_ints = 0;
    uint8_t * smp_ws = nullptr;
    size_t smp_ws_size = 0;
    ggml_backend_buffer_type buft{};
    char name[64] = { 0 };
};

std::vector<hip_device> & devices() {
    static std::vector<hip_device> d(16);
    return d;
}

int device_count() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void) hipGetLastError();
        return 0;
    }
    return n;
}

hip_device & dev(int id) {
    hip_device & d = devices()[id];
    if (!d.ready) {
        HIP_CHECK(hipSetDevice(id));
        // default priority on purpose: streams of different priorities are not mixed here
        HIP_CHECK(hipStreamCreateWithFlags(&d.stream, hipStreamNonBlocking));
        d.id = id;
        d.ready = true;
    }
    HIP_CHECK(hipSetDevice(id));
    return d;
}

uint8_t * staging(hip_device & d, size_t size) {
    if (size > d.staging_size) {
        if (d.staging) HIP_CHECK(hipFree(d.staging));
        d.staging_size = std::max(size, (size_t) 1 << 24);
        HIP_CHECK(hipMalloc(&d.staging, d.staging_size));
    }
    return d.staging;
}

constexpr size_t UP_RING = (size_t) 4 << 20;        // bytes of the upload ring
constexpr size_t UP_SMALL = (size_t) 256 << 10;      // uploads up to this size go through the ring
constexpr size_t DOWN_MAX = (size_t) 16 << 20;       // downloads up to this size land in pinned memory

// the stream has no queued work left: the upload ring can be reused from its start
void drained(hip_device & d) { d.up_off = 0; }

// a slot of the upload ring for size bytes, or nullptr when it does not fit before the stream drains
uint8_t * upload_slot(hip_device & d, size_t size) {
    if (size > UP_SMALL) return nullptr;
    if (!d.up_ring) HIP_CHECK(hipHostMalloc((void **) &d.up_ring, UP_RING, hipHostMallocDefault));
    const size_t off = (d.up_off + 255) & ~(size_t) 255;
    if (off + size > UP_RING) return nullptr;
    d.up_off = off + size;
    return d.up_ring + off;
}

uint8_t * download_area(hip_device & d, size_t size) {
    if (size > DOWN_MAX) return nullptr;
    if (size > d.down_size) {
        if (d.down) HIP_CHECK(hipHostFree(d.down));
        d.down_size = std::max(size, (size_t) 1 << 20);
        HIP_CHECK(hipHostMalloc((void **) &d.down, d.down_size, hipHostMallocDefault));
    }
    return d.down;
}

bool is_repacked(int type) { return type == GGML_TYPE_Q4_0 || type == GGML_TYPE_Q8_0 || type == GGML_TYPE_Q6_K; }
int qs_bytes_of(int type) { return type == GGML_TYPE_Q4_0 ? Q4_0_QS : type == GGML_TYPE_Q8_0 ? Q8_0_QS : 128; }

// planes of a repacked tensor: base allocation (view_src or self) and the block index of t.
// Q4_0 / Q8_0: [qs][d]; Q6_K: [ql = qs][qh][sc][d] (q6k_planes)
struct planes {
    uint8_t * qs;
    __half * d;
    uint8_t * qh;         // Q6_K
    int8_t * sc;          // Q6_K
    int64_t first_block;  // block index of t->data within the base tensor
    int64_t base_blocks;
};

planes planes_of(const ggml_tensor * t) {
    const ggml_tensor * base = t->view_src ? t->view_src : t;
    const size_t bs = ggml_type_size(t->type);
    planes p;
    p.base_blocks = (int64_t) (ggml_nbytes(base) / bs);
    uint8_t * b0 = (uint8_t *) base->data;
    p.qs = b0;
    p.qh = nullptr;
    p.sc = nullptr;
    if (t->type == GGML_TYPE_Q6_K) {
        p.qh = b0 + p.base_blocks * 128;
        p.sc = (int8_t *) (b0 + p.base_blocks * 192);
        p.d = (__half *) (b0 + p.base_blocks * 208);
    } else {
        p.d = (__half *) (b0 + p.base_blocks * qs_bytes_of(t->type));
    }
    const size_t off = (size_t) ((const char *) t->data - (const char *) base->data);
    if (off % bs) HIP_ABORT("tensor '%s': view offset is not block aligned", t->name);
    p.first_block = (int64_t) (off / bs);
    return p;
}

q6k_planes q6k_of(const planes & p) { return q6k_planes{ p.qs, p.qh, p.sc, p.d }; }

void repack_blocks(const ggml_tensor * t, const planes & p, const uint8_t * raw, int64_t nblocks, int64_t first, hipStream_t st) {
    if (t->type == GGML_TYPE_Q6_K) launch_repack_q6k(raw, q6k_of(p), nblocks, first, st);
    else launch_repack_q(t->type, raw, p.qs, p.d, nblocks, first, st);
}

void unpack_blocks(const ggml_tensor * t, const planes & p, uint8_t * raw, int64_t nblocks, int64_t first, hipStream_t st) {
    if (t->type == GGML_TYPE_Q6_K) launch_unpack_q6k(raw, q6k_of(p), nblocks, first, st);
    else launch_unpack_q(t->type, raw, p.qs, p.d, nblocks, first, st);
}

// ---------------------------------------------------------------------------------------------
// buffers

struct buf_ctx {
    int device;
    void * base;
};

void buf_free(ggml_backend_buffer_t b) {
    buf_ctx * c = (buf_ctx *) b->context;
    // queued kernels may still use the buffer (asynchronous graph computes)
    HIP_CHECK(hipStreamSynchronize(dev(c->device).stream));
    HIP_CHECK(hipFree(c->base));
    delete c;
}

void * buf_base(ggml_backend_buffer_t b) { return ((buf_ctx *) b->context)->base; }

void buf_set(ggml_backend_buffer_t b, ggml_tensor * t, const void * data, size_t off, size_t size) {
    hip_device & d = dev(((buf_ctx *) b->context)->device);
    if (is_repacked(t->type)) {
        const size_t bs = ggml_type_size(t->type);
        if (off % bs || size % bs) HIP_ABORT("tensor_set on '%s': partial block write", t->name);
        const planes p = planes_of(t);
        const size_t chunk = (size_t) (64u << 20) / bs * bs;
        for (size_t done = 0; done < size; done += chunk) {
            const size_t n = std::min(chunk, size - done);
            uint8_t * st = staging(d, n);
            HIP_CHECK(hipMemcpyAsync(st, (const uint8_t *) data + done, n, hipMemcpyHostToDevice, d.stream));
            repack_blocks(t, p, st, (int64_t) (n / bs), p.first_block + (int64_t) ((off + done) / bs), d.stream);
            HIP_CHECK(hipStreamSynchronize(d.stream));
            drained(d);
        }
        return;
    }
    if (uint8_t * slot = upload_slot(d, size)) {
        // the caller's bytes are copied now; the device copy is ordered before later work on the stream
        memcpy(slot, data, size);
        HIP_CHECK(hipMemcpyAsync((char *) t->data + off, slot, size, hipMemcpyHostToDevice, d.stream));
        return;
    }
    HIP_CHECK(hipMemcpyAsync((char *) t->data + off, data, size, hipMemcpyHostToDevice, d.stream));
    HIP_CHECK(hipStreamSynchronize(d.stream));
    drained(d);
}

void buf_get(ggml_backend_buffer_t b, const ggml_tensor * t, void * data, size_t off, size_t size) {
    hip_device & d = dev(((buf_ctx *) b->context)->device);
    if (is_repacked(t->type)) {
        const size_t bs = ggml_type_size(t->type);
        if (off % bs || size % bs) HIP_ABORT("tensor_get on '%s': partial block read", t->name);
        const planes p = planes_of(t);
        const size_t chunk = (size_t) (64u << 20) / bs * bs;
        for (size_t done = 0; done < size; done += chunk) {
            const size_t n = std::min(chunk, size - done);
            uint8_t * st = staging(d, n);
            unpack_blocks(t, p, st, (int64_t) (n / bs), p.first_block + (int64_t) ((off + done) / bs), d.stream);
            HIP_CHECK(hipMemcpyAsync((uint8_t *) data + done, st, n, hipMemcpyDeviceToHost, d.stream));
            HIP_CHECK(hipStreamSynchronize(d.stream));
            drained(d);
        }
        return;
    }
    if (uint8_t * area = download_area(d, size)) {
        HIP_CHECK(hipMemcpyAsync(area, (const char *) t->data + off, size, hipMemcpyDeviceToHost, d.stream));
        HIP_CHECK(hipStreamSynchronize(d.stream));
        drained(d);
        memcpy(data, area, size);
        return;
    }
    HIP_CHECK(hipMemcpyAsync(data, (const char *) t->data + off, size, hipMemcpyDeviceToHost, d.stream));
    HIP_CHECK(hipStreamSynchronize(d.stream));
    drained(d);
}

void buf_memset(ggml_backend_buffer_t b, ggml_tensor * t, uint8_t v, size_t off, size_t size) {
    hip_device & d = dev(((buf_ctx *) b->context)->device);
    if (is_repacked(t->type) && v != 0) HIP_ABORT("tensor_memset on '%s': only zero fills are supported for %s", t->name, ggml_type_name(t->type));
    if (is_repacked(t->type)) {
        const size_t bs = ggml_type_size(t->type);
        if (off % bs || size % bs) HIP_ABORT("tensor_memset on '%s': partial block", t->name);
        const planes p = planes_of(t);
        const int64_t b0 = p.first_block + (int64_t) (off / bs), nb = (int64_t) (size / bs);
        HIP_CHECK(hipMemsetAsync(p.qs + b0 * qs_bytes_of(t->type), 0, nb * qs_bytes_of(t->type), d.stream));
        HIP_CHECK(hipMemsetAsync(p.d + b0, 0, nb * sizeof(__half), d.stream));
        if (t->type == GGML_TYPE_Q6_K) {
            HIP_CHECK(hipMemsetAsync(p.qh + b0 * 64, 0, nb * 64, d.stream));
            HIP_CHECK(hipMemsetAsync(p.sc + b0 * 16, 0, nb * 16, d.stream));
        }
    } else {
        HIP_CHECK(hipMemsetAsync((char *) t->data + off, v, size, d.stream));
    }
    HIP_CHECK(hipStreamSynchronize(d.stream));
    drained(d);
}

void buf_clear(ggml_backend_buffer_t b, uint8_t v) {
    buf_ctx * c = (buf_ctx *) b->context;
    hip_device & d = dev(c->device);
    HIP_CHECK(hipMemsetAsync(c->base, v, b->size, d.stream));
    HIP_CHECK(hipStreamSynchronize(d.stream));
    drained(d);
}

const char * buft_name(ggml_backend_buffer_type_t t) { return ((hip_device *) t->context)->name; }
size_t buft_align(ggml_backend_buffer_type_t) { return 256; }
bool buft_is_host(ggml_backend_buffer_type_t) { return false; }
bool buft_no_reuse(ggml_backend_buffer_type_t) { return true; }

ggml_backend_buffer_t buft_alloc(ggml_backend_buffer_type_t t, size_t size) {
    hip_device & d = dev(((hip_device *) t->context)->id);
    void * p = nullptr;
    if (hipMalloc(&p, std::max<size_t>(size, 256)) != hipSuccess) {
        (void) hipGetLastError();
        fprintf(stderr, "ggml-hip: failed to allocate %.1f MiB on device %d\n", size / 1048576.0, d.id);
        return nullptr;
    }
    buf_ctx * c = new buf_ctx{ d.id, p };
    ggml_backend_buffer_i iface = { buf_free, buf_base, nullptr, buf_set, buf_get, buf_memset, buf_clear };
    return ggml_backend_buffer_init(t, iface, c, size);
}

// ---------------------------------------------------------------------------------------------
// backend context

struct prof_entry { int64_t launches = 0; double ms = 0.0; double bytes = 0.0; };

struct pending_event { std::string name; double bytes; hipEvent_t a, b; };

// thrown by a fixed arena (graph_compute_static) when a compute needs more than it holds
struct scratch_overflow {
    size_t needed;
};

struct scratch_arena {
    std::vector<std::pair<uint8_t *, size_t>> chunks;
    size_t chunk = 0, off = 0;
    bool fixed = false;          // one caller-provided chunk, never grown (no allocation)
    void reset() { chunk = 0; off = 0; }
    void * alloc(size_t size) {
        size = (size + 255) & ~(size_t) 255;
        while (chunk < chunks.size() && off + size > chunks[chunk].second) { chunk++; off = 0; }
        if (chunk == chunks.size() && fixed) throw scratch_overflow{ chunks.empty() ? size : chunks[0].second + size };
        if (chunk == chunks.size()) {
            const size_t cap = std::max(size, (size_t) 64 << 20);
            uint8_t * p = nullptr;
            HIP_CHECK(hipMalloc(&p, cap));
            chunks.push_back({ p, cap });
            off = 0;
        }
        void * r = chunks[chunk].first + off;
        off += size;
        return r;
    }
    void release() {
        if (!fixed) {
            for (auto & c : chunks) HIP_CHECK(hipFree(c.first));
        }
        chunks.clear();
        reset();
    }
};

struct act_entry {       // quantized copy of an activation tensor
    int kind;            // 1 = q8 (Q8_0 semantics), 2 = q8K
    q8_act q8;
    q8k_act q8k;
    int64_t K, ncols;
};

// fusion switches (all on by default; GGML_HIP_FUSE=<bitmask> narrows them for A/B runs)
enum fuse_bits {
    FUSE_NORM   = 1,   // rms_norm -> mul(weight) [+ activation quantization]
    FUSE_GROUP  = 2,   // mul_mats sharing one input in one launch
    FUSE_SWIGLU = 4,   // gate/up -> silu -> mul in the GEMV epilogue
    FUSE_ADD    = 8,   // residual add in the GEMV epilogue
    FUSE_ATTN   = 16,  // split-KV decode attention
    FUSE_ACTQ   = 32,  // producers emit the Q8 activation their GEMV consumers read
    FUSE_NORMQ  = 64,  // rms_norm * w folded into the prologue of the GEMVs that consume it
    FUSE_ROPE   = 128, // RoPE stored straight into the KV cache; independent RoPE/copies in one launch
    FUSE_ROUTE  = 256, // MoE router softmax -> top-k -> renormalized weights in one launch
    FUSE_MC     = 512, // several activation columns per GEMV workgroup; mul_mat_id grouped by expert
    FUSE_ROUTEG = 1024, // one token's MoE routing inside its routed gate/up GEMV launch
    FUSE_ACCO   = 2048, // one-query attention output accumulated by PV, read as doubles by its GEMVs
    FUSE_WSUMQ  = 4096, // MoE weighted sum also writes the next rms_norm * w as Q8_K (several tokens)
    FUSE_ALL    = 8191,
};

struct hip_backend_ctx {
    int device = 0;
    bool fusion = true;
    int fuse_mask = FUSE_ALL;
    bool profiling = false;
    int profile_every = 1;           // time one graph compute in every profile_every
    int64_t computes = 0;
    bool timing = false;             // this compute is timed
    std::string profile_filter;      // only kernels whose name starts with this get events
    ggml_backend_eval_callback cb = nullptr;
    void * cb_user = nullptr;
    scratch_arena scratch;
    std::map<std::string, prof_entry> prof;
    std::vector<pending_event> pending;
    std::vector<hipEvent_t> event_pool;
    size_t event_next = 0;
};

// ---------------------------------------------------------------------------------------------
// graph executor

tview tv(const ggml_tensor * t) {
    tview v;
    v.data = (char *) t->data;
    v.type = t->type;
    for (int i = 0; i < 4; i++) { v.ne[i] = t->ne[i]; v.nb[i] = (int64_t) t->nb[i]; }
    return v;
}

// profile names of the GEMV launches, by weight type
const char * gemv_prof_name(int wtype, bool swiglu) {
    switch (wtype) {
        case GGML_TYPE_Q4_0: return swiglu ? "gemv_q4_0_swiglu" : "gemv_q4_0";
        case GGML_TYPE_Q8_0: return swiglu ? "gemv_q8_0_swiglu" : "gemv_q8_0";
        case GGML_TYPE_Q5_K: return swiglu ? "gemv_q5_K_swiglu" : "gemv_q5_K";
        case GGML_TYPE_Q6_K: return swiglu ? "gemv_q6_K_swiglu" : "gemv_q6_K";
        default: return swiglu ? "gemv_q4_K_swiglu" : "gemv_q4_K";
    }
}

int dot_kind(int wtype) {
    if (wtype == GGML_TYPE_Q4_0 || wtype == GGML_TYPE_Q8_0) return 1;
    if (is_kquant(wtype)) return 2;
    return 0;
}

bool is_2d_contig(const ggml_tensor * t) { return t->ne[2] == 1 && t->ne[3] == 1 && ggml_is_contiguous(t); }

// the nodes of one decode-attention chain (anchored at the K^T Q mul_mat)
struct attn_match {
    int kq = -1, sm = -1, vt = -1, kqv = -1, pm = -1, ct = -1;
    const ggml_tensor * kp = nullptr;   // permuted K cache view [hd, n_kv, n_head_kv]
    const ggml_tensor * qp = nullptr;   // permuted Q [hd, n_q, n_head]
    const ggml_tensor * vp = nullptr;   // permuted V cache view [n_kv, hd, n_head_kv]
    const ggml_tensor * mask = nullptr;
    float scale = 1.0f;
};

class executor {
public:
    executor(hip_backend_ctx & ctx, ggml_cgraph * g) : c_(ctx), g_(g), st_(dev(ctx.device).stream) {}

    void run() {
        c_.scratch.reset();
        index_graph();
        done_.assign(g_->n_nodes, false);
        attn_.clear();
        norm_.clear();
        act_.clear();
        pending_route_.clear();
        // plan the attention fusions first: the V^T copy precedes K^T Q in node order and must
        // not run when the chain is replaced
        if (fuse(FUSE_ATTN)) {
            for (int i = 0; i < g_->n_nodes; i++) {
                attn_match m;
                if (g_->nodes[i]->op == GGML_OP_MUL_MAT && match_attention(i, m)) {
                    attn_[i] = m;
                    done_[m.vt] = true;
                }
            }
        }
        for (int i = 0; i < g_->n_nodes; i++) {
            if (done_[i]) continue;
            wrote_.clear();
            if (c_.profiling && !c_.timing) {
                // host time per handled node, by op ("host_op:<op>" entries of a profiled compute
                // without events: a timed one also waits for the device)
                const auto h0 = std::chrono::steady_clock::now();
                exec_node(i);
                prof_entry & e = c_.prof[std::string("host_op:") + ggml_op_name(g_->nodes[i]->op)];
                e.launches++;
                e.ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - h0).count();
            } else {
                exec_node(i);
            }
            done_[i] = true;
            if (c_.cb) report();
        }
        if (!pending_route_.empty()) HIP_ABORT("a held-back MoE routing was never run");
    }

private:
    hip_backend_ctx & c_;
    ggml_cgraph * g_;
    hipStream_t st_;
    std::unordered_map<const ggml_tensor *, int> idx_;
    std::vector<std::vector<int>> users_;
    std::vector<bool> done_;
    std::unordered_map<const ggml_tensor *, act_entry> act_;
    std::unordered_map<const ggml_tensor *, gemv_norm> norm_;   // deferred rms_norm * w outputs
    std::unordered_map<int, attn_match> attn_;
    std::unordered_map<int, int> silu_of_;    // mul node -> its held-back silu node (op_swiglu)
    struct router_norm { int norm, mul; float eps; };
    std::unordered_map<int, router_norm> router_norm_;   // router mul_mat node -> the norm it computes
    // one-token routings held back by op_moe_route, keyed by the ids view the mul_mat_ids read
    std::unordered_map<const ggml_tensor *, moe_route> pending_route_;
    std::vector<const ggml_tensor *> wrote_;

    bool fuse(int bit) const { return c_.fusion && (c_.fuse_mask & bit); }

    void report() {
        HIP_CHECK(hipStreamSynchronize(st_));
        for (const ggml_tensor * t : wrote_) {
            if (!c_.cb((ggml_tensor *) t, false, c_.cb_user)) { c_.cb = nullptr; return; }
        }
    }

    // ---- graph structure ----
    void index_graph() {
        idx_.clear();
        idx_.reserve(g_->n_nodes * 2);
        for (int i = 0; i < g_->n_nodes; i++) idx_[g_->nodes[i]] = i;
        users_.assign(g_->n_nodes, {});
        for (int i = 0; i < g_->n_nodes; i++) {
            const ggml_tensor * n = g_->nodes[i];
            for (int s = 0; s < GGML_MAX_SRC; s++) {
                if (!n->src[s]) continue;
                bool dup = false;
                for (int r = 0; r < s; r++) dup = dup || n->src[r] == n->src[s];
                if (dup) continue;
                auto it = idx_.find(n->src[s]);
                if (it != idx_.end()) users_[it->second].push_back(i);
            }
        }
    }
    int node_index(const ggml_tensor * t) const {
        auto it = idx_.find(t);
        return it == idx_.end() ? -1 : it->second;
    }
    bool is_output(int i) const { return i == g_->n_nodes - 1 || (g_->nodes[i]->flags & GGML_TENSOR_FLAG_OUTPUT); }
    // the single consumer of node i, or -1 (0 or >1 users, or a graph output)
    int sole_user(int i) const {
        if (i < 0 || is_output(i) || users_[i].size() != 1) return -1;
        return users_[i][0];
    }

    // ---- profiling ----
    hipEvent_t event() {
        if (c_.event_next == c_.event_pool.size()) {
            hipEvent_t e;
            HIP_CHECK(hipEventCreate(&e));
            c_.event_pool.push_back(e);
        }
        return c_.event_pool[c_.event_next++];
    }
    // times the kernels launched while it lives (one op) through their dispatch timestamps
    struct prof_scope {
        executor * ex;
        const char * name;
        double bytes;
        bool on = false;
        prof_scope(executor * e, const char * n, double b) : ex(e), name(n), bytes(b) {
            if (ex->c_.timing && ex->c_.profile_filter.compare(0, ex->c_.profile_filter.size(), n, 0,
                                                                  ex->c_.profile_filter.size()) == 0) {
                g_launch_timing = launch_timing{ ex->event(), ex->event(), 0 };
                on = true;
            }
        }
        ~prof_scope() {
            if (!on) return;
            const launch_timing t = g_launch_timing;
            g_launch_timing = launch_timing{};
            if (t.launches > 0) ex->c_.pending.push_back({ name, bytes, t.start, t.stop });
        }
    };

    // ---- activation quantization ----
    const act_entry * ensure_act(const ggml_tensor * x, int kind) {
        auto it = act_.find(x);
        if (it != act_.end() && it->second.kind == kind) return &it->second;
        const int64_t K = x->ne[0], ncols = ggml_nrows(x);
        if (x->type != GGML_TYPE_F32 || x->nb[0] != sizeof(float) ||
            (x->ne[2] > 1 && x->nb[2] != x->nb[1] * x->ne[1]) || (x->ne[3] > 1 && x->nb[3] != x->nb[2] * x->ne[2])) {
            HIP_ABORT("activation '%s' for a quantized mul_mat: rows must be f32 and evenly strided", x->name);
        }
        act_entry e = alloc_act(kind, K, ncols);
        const int64_t col_stride = (int64_t) (x->nb[1] / sizeof(float));
        if (kind == 1) {
            prof_scope ps(this, "quantize_q8", (double) (K * ncols * 4));
            launch_quantize_q8((const float *) x->data, col_stride, K, ncols, e.q8, st_);
        } else {
            prof_scope ps(this, "quantize_q8K", (double) (K * ncols * 4));
            launch_quantize_q8k((const float *) x->data, col_stride, K, ncols, e.q8k, st_);
        }
        act_[x] = e;
        return &act_[x];
    }
    act_entry alloc_act(int kind, int64_t K, int64_t ncols) {
        act_entry e{};
        e.kind = kind;
        e.K = K;
        e.ncols = ncols;
        if (kind == 1) {
            e.q8.qs = (int8_t *) c_.scratch.alloc((size_t) (K * ncols));
            e.q8.d = (float *) c_.scratch.alloc((size_t) (K / 32 * ncols) * 4);
            e.q8.s = (int32_t *) c_.scratch.alloc((size_t) (K / 32 * ncols) * 4);
        } else {
            e.q8k.qs = (int8_t *) c_.scratch.alloc((size_t) (K * ncols));
            e.q8k.d = (float *) c_.scratch.alloc((size_t) (K / 256 * ncols) * 4);
            e.q8k.bsums = (int16_t *) c_.scratch.alloc((size_t) (K / 16 * ncols) * 2);
        }
        return e;
    }
    // the quantized form all consumers of node i want (0: none / mixed / not all quantized mul_mats)
    int wanted_act_kind(int i) const {
        if (!fuse(FUSE_ACTQ) || i < 0 || users_[i].empty()) return 0;
        int kind = 0;
        for (int u : users_[i]) {
            const ggml_tensor * n = g_->nodes[u];
            if (n->op != GGML_OP_MUL_MAT || n->src[1] != g_->nodes[i]) return 0;
            const int k = dot_kind(n->src[0]->type);
            if (k == 0 || (kind && k != kind)) return 0;
            kind = k;
        }
        return kind;
    }

    // the weight type of the quantized GEMVs that are node u's only consumers (-1: some consumer is
    // not such a GEMV, or they mix dot types)
    int gemv_only_consumers(int u) const {
        if (users_[u].empty()) return -1;
        const ggml_tensor * m = g_->nodes[u];
        int wtype = -1;
        for (int j : users_[u]) {
            const ggml_tensor * n = g_->nodes[j];
            if ((n->op != GGML_OP_MUL_MAT && n->op != GGML_OP_MUL_MAT_ID) || n->src[1] != m || n->src[0] == m || attn_.count(j) ||
                !gemv_capable(n)) return -1;
            if (wtype >= 0 && dot_kind(n->src[0]->type) != dot_kind(wtype)) return -1;
            wtype = n->src[0]->type;
        }
        return wtype;
    }

    int64_t max_consumer_rows(int u) const {
        int64_t r = 0;
        for (int j : users_[u]) r = std::max(r, (int64_t) g_->nodes[j]->src[0]->ne[1]);
        return r;
    }

    // rms_norm * w (node u, rows of N) whose every consumer is a quantized GEMV that can compute the
    // normalization in its prologue: the normalized activation is then never materialized
    bool norm_deferrable(int u, int64_t N) const {
        if (!fuse(FUSE_NORMQ) || !fuse(FUSE_ACTQ) || is_output(u)) return false;
        const int wtype = gemv_only_consumers(u);
        return wtype >= 0 && N <= gemv_prologue_max_k(wtype, true);
    }

    // ---- dispatch ----
    void exec_node(int i) {
        ggml_tensor * n = g_->nodes[i];
        switch (n->op) {
            case GGML_OP_NONE: case GGML_OP_RESHAPE: case GGML_OP_VIEW: case GGML_OP_PERMUTE: case GGML_OP_TRANSPOSE:
                return;
            case GGML_OP_RMS_NORM: op_rms_norm(i); return;
            case GGML_OP_ROPE: op_rope(i); return;
            case GGML_OP_MUL_MAT: op_mul_mat(i); return;
            case GGML_OP_MUL_MAT_ID:
                if (!gemv_capable(n)) HIP_ABORT("mul_mat_id '%s': unsupported operands", n->name);
                op_gemv(i);
                return;
            case GGML_OP_MUL:
                // a mul whose silu operand was held back runs as the fused SwiGLU (nothing else
                // may take it: the silu output was never written)
                if (silu_of_.count(i)) { run_swiglu(silu_of_[i], i); return; }
                if (fuse(FUSE_ADD) && op_moe_wsum(i)) return;
                break;
            case GGML_OP_SOFT_MAX:
                if (fuse(FUSE_ROUTE) && op_moe_route(i)) return;
                break;
            case GGML_OP_UNARY:
                if (fuse(FUSE_SWIGLU) && op_swiglu(i)) return;
                break;
            default: break;
        }
        wrote_.push_back(n);
        switch (n->op) {
            case GGML_OP_GET_ROWS: op_get_rows(n); return;
            case GGML_OP_ADD: { prof_scope ps(this, "add", 0); launch_binary(0, tv(n->src[0]), tv(n->src[1]), tv(n), st_); return; }
            case GGML_OP_MUL: { prof_scope ps(this, "mul", 0); launch_binary(1, tv(n->src[0]), tv(n->src[1]), tv(n), st_); return; }
            case GGML_OP_DIV: { prof_scope ps(this, "div", 0); launch_binary(2, tv(n->src[0]), tv(n->src[1]), tv(n), st_); return; }
            case GGML_OP_SUB: { prof_scope ps(this, "sub", 0); launch_binary(3, tv(n->src[0]), tv(n->src[1]), tv(n), st_); return; }
            case GGML_OP_L2_NORM: {
                float eps;
                memcpy(&eps, n->op_params, 4);
                prof_scope ps(this, "l2_norm", 0);
                launch_l2_norm(tv(n->src[0]), tv(n), eps, st_);
                return;
            }
            case GGML_OP_CONCAT: {
                if (n->type != GGML_TYPE_F32 && n->type != GGML_TYPE_F16 && n->type != GGML_TYPE_I32) HIP_ABORT("concat of type %d", n->type);
                prof_scope ps(this, "concat", 0);
                launch_concat(tv(n->src[0]), tv(n->src[1]), tv(n), n->op_params[0], st_);
                return;
            }
            case GGML_OP_GLU: {
                if (n->op_params[0] != GGML_GLU_OP_SWIGLU) HIP_ABORT("unsupported glu op %d", n->op_params[0]);
                prof_scope ps(this, "glu", 0);
                launch_glu(tv(n->src[0]), tv(n->src[1]), tv(n), st_);
                return;
            }
            case GGML_OP_SUM_ROWS: { prof_scope ps(this, "sum_rows", 0); launch_sum_rows(tv(n->src[0]), tv(n), st_); return; }
            case GGML_OP_ARGSORT: {
                prof_scope ps(this, "argsort", 0);
                launch_argsort(tv(n->src[0]), tv(n), n->op_params[0] == GGML_SORT_ORDER_DESC, st_);
                return;
            }
            case GGML_OP_SCALE: {
                float s;
                memcpy(&s, n->op_params, 4);
                prof_scope ps(this, "scale", 0);
                launch_unary(4, s, tv(n->src[0]), tv(n), st_);
                return;
            }
            case GGML_OP_SQR: { prof_scope ps(this, "sqr", 0); launch_unary(3, 0, tv(n->src[0]), tv(n), st_); return; }
            case GGML_OP_UNARY: {
                const int u = n->op_params[0];
                const int op = u == GGML_UNARY_OP_SILU ? 0 : u == GGML_UNARY_OP_RELU ? 1 : u == GGML_UNARY_OP_SIGMOID ? 2 :
                               u == GGML_UNARY_OP_ABS ? 5 : u == GGML_UNARY_OP_SOFTPLUS ? 6 : -1;
                if (op < 0) HIP_ABORT("unsupported unary op %d", u);
                prof_scope ps(this, "unary", 0);
                launch_unary(op, 0, tv(n->src[0]), tv(n), st_);
                return;
            }
            case GGML_OP_CPY: case GGML_OP_CONT: case GGML_OP_DUP: {
                if (ggml_is_quantized(n->type) || ggml_is_quantized(n->src[0]->type)) HIP_ABORT("copy of quantized tensor '%s'", n->name);
                prof_scope ps(this, "cpy", (double) (ggml_nbytes(n->src[0]) + ggml_nbytes(n)));
                launch_cpy(tv(n->src[0]), tv(n), st_);
                return;
            }

            case GGML_OP_SOFT_MAX: {
                float scale, max_bias;
                memcpy(&scale, &n->op_params[0], 4);
                memcpy(&max_bias, &n->op_params[1], 4);
                tview m{};
                if (n->src[1]) m = tv(n->src[1]);
                prof_scope ps(this, "soft_max", 0);
                launch_soft_max(tv(n->src[0]), n->src[1] ? &m : nullptr, tv(n), scale, max_bias, st_);
                return;
            }
            case GGML_OP_FLASH_ATTN_EXT: op_flash_attn(n); return;
            case GGML_OP_ARGMAX: {
                prof_scope ps(this, "argmax", 0);
                const tview a = tv(n->src[0]);
                if (a.ne[1] == 1 && a.ne[0] >= ARGMAX_ROW_MIN) {
                    float * pv = (float *) c_.scratch.alloc(ARGMAX_PARTS * sizeof(float));
                    int * pi = (int *) c_.scratch.alloc(ARGMAX_PARTS * sizeof(int));
                    // copies of the one index into I32 cells (the decode loop's next token and its
                    // history slot): written by the final launch instead of two copy launches
                    int32_t * extra[2] = { nullptr, nullptr };
                    int ne = 0;
                    if (fuse(FUSE_ADD) && !c_.cb) {
                        for (int u : users_[i]) {
                            const ggml_tensor * c = g_->nodes[u];
                            if (c->op != GGML_OP_CPY || c->src[0] != n || c->type != GGML_TYPE_I32 || ggml_nelements(c) != 1 ||
                                ne == 2 || done_[u]) { ne = -1; break; }
                            extra[ne++] = (int32_t *) c->data;
                        }
                        if (ne > 0) {
                            for (int u : users_[i]) {
                                done_[u] = true;
                                wrote_.push_back(g_->nodes[u]);
                            }
                        } else {
                            extra[0] = extra[1] = nullptr;
                        }
                    }
                    launch_argmax_row(a, (int32_t *) n->data, pv, pi, st_, extra[0], extra[1]);
                } else {
                    launch_argmax(a, (int32_t *) n->data, st_);
                }
                return;
            }
            default:
                HIP_ABORT("op %s is not supported by the hip backend (node '%s')", ggml_op_name(n->op), n->name);
        }
    }

    void op_get_rows(ggml_tensor * n) {
        const ggml_tensor * a = n->src[0];
        planes p{};
        if (is_repacked(a->type)) p = planes_of(a);
        prof_scope ps(this, "get_rows", (double) ggml_nbytes(n));
        launch_get_rows(tv(a), tv(n->src[1]), tv(n), p.qs, p.d, q6k_of(p), p.first_block, st_);
    }

    static bool is_view_op(int op) {
        return op == GGML_OP_NONE || op == GGML_OP_RESHAPE || op == GGML_OP_VIEW || op == GGML_OP_PERMUTE ||
               op == GGML_OP_TRANSPOSE;
    }
    // the data of t is final before the next launch: a leaf, a finished node, or a view of one
    bool ready(const ggml_tensor * t) const {
        const int k = node_index(t);
        if (k < 0 || done_[k]) return true;
        return is_view_op(t->op) && t->src[0] && ready(t->src[0]);
    }

    static rope_params rope_params_of(const ggml_tensor * n) {
        rope_params p{};
        p.n_dims = n->op_params[1];
        p.mode = n->op_params[2];
        const int n_ctx_orig = n->op_params[4];
        float freq_base, beta_fast, beta_slow;
        memcpy(&freq_base, n->op_params + 5, 4);
        memcpy(&p.freq_scale, n->op_params + 6, 4);
        memcpy(&p.ext_factor, n->op_params + 7, 4);
        memcpy(&p.attn_factor, n->op_params + 8, 4);
        memcpy(&beta_fast, n->op_params + 9, 4);
        memcpy(&beta_slow, n->op_params + 10, 4);
        ggml_rope_yarn_corr_dims(p.n_dims, n_ctx_orig, freq_base, beta_fast, beta_slow, p.corr_dims);
        p.theta_scale = powf(freq_base, -2.0f / p.n_dims);
        return p;
    }

    // RoPE node i as a job; when its only consumer copies it into an F16/F32 tensor of the same shape
    // (the KV cache append), the rotation is stored there directly
    void add_rope_job(rope_batch & B, std::vector<int> & members, int i) {
        ggml_tensor * n = g_->nodes[i];
        if (n->src[0]->type != GGML_TYPE_F32 || n->type != GGML_TYPE_F32) HIP_ABORT("rope: f32 only");
        ggml_tensor * dst = n;
        const int u = fuse(FUSE_ROPE) ? sole_user(i) : -1;
        if (u >= 0) {
            ggml_tensor * c = g_->nodes[u];
            if (c->op == GGML_OP_CPY && c->src[0] == n && (c->type == GGML_TYPE_F16 || c->type == GGML_TYPE_F32) &&
                ggml_are_same_shape(n, c)) {
                dst = c;
                members.push_back(u);
            }
        }
        B.job[B.n_jobs++] = rope_job{ tv(n->src[0]), tv(dst), (const int32_t *) n->src[1]->data,
                                      n->src[2] ? (const float *) n->src[2]->data : nullptr, rope_params_of(n),
                                      ggml_nelements(n->src[0]) / 2 };
        members.push_back(i);
        wrote_.push_back(dst);
    }

    // RoPE node i, launched together with the RoPE nodes and F32 -> F16/F32 copies that follow it
    // in the graph and whose inputs are already final (the window holds views, RoPEs and copies
    // only, none of which reads what another writes)
    // rms_norm * w outputs held back for a RoPE (QK-Norm)
    struct pending_norm { const ggml_tensor * x; const ggml_tensor * w; float eps; };
    std::unordered_map<const ggml_tensor *, pending_norm> pnorm_;

    // A per-head rms_norm * w (QK-Norm) read only by a RoPE: held back until that RoPE's batch is
    // placed (folded into the attention, or run just before the RoPE). Launches nothing.
    bool defer_qk_norm(int i) {
        const ggml_tensor * n = g_->nodes[i];
        const ggml_tensor * x = n->src[0];
        if (!fuse(FUSE_NORM) || !fuse(FUSE_ROPE) || !fuse(FUSE_ATTN) || n->op != GGML_OP_RMS_NORM) return false;
        if (x->type != GGML_TYPE_F32 || !ggml_is_contiguous(x) || !ggml_is_contiguous(n) || x->ne[0] > 256 ||
            x->ne[3] != 1) return false;
        const int u = sole_user(i);
        if (u < 0) return false;
        const ggml_tensor * m = g_->nodes[u];
        const ggml_tensor * w = m->src[1];
        if (m->op != GGML_OP_MUL || m->src[0] != n || w->type != GGML_TYPE_F32 || ggml_nrows(w) != 1 ||
            w->ne[0] != x->ne[0] || !ggml_is_contiguous(w) || !ggml_is_contiguous(m)) return false;
        const int r = sole_user(u);
        if (r < 0 || g_->nodes[r]->op != GGML_OP_ROPE || g_->nodes[r]->src[0] != m) return false;
        float eps;
        memcpy(&eps, n->op_params, 4);
        pnorm_[m] = pending_norm{ x, w, eps };
        done_[u] = true;
        return true;
    }

    void materialize_norm(const ggml_tensor * m) {
        auto it = pnorm_.find(m);
        if (it == pnorm_.end()) return;
        const pending_norm pn = it->second;
        pnorm_.erase(it);
        const int64_t N = pn.x->ne[0], rows = ggml_nrows(pn.x);
        prof_scope ps(this, "rms_norm_mul", (double) (N * rows * 8 + N * 4));
        launch_rms_norm((const float *) pn.x->data, N, (const float *) pn.w->data, (float *) m->data, N, N, rows, pn.eps,
                        nullptr, nullptr, st_);
        wrote_.push_back(m);
    }

    qk_norm qk_norm_of(const ggml_tensor * m) {
        auto it = pnorm_.find(m);
        if (it == pnorm_.end()) return qk_norm{};
        const pending_norm pn = it->second;
        pnorm_.erase(it);
        return qk_norm{ (const float *) pn.x->data, (int64_t) (pn.x->nb[1] / sizeof(float)), (int64_t) (pn.x->nb[2] / sizeof(float)),
                        (const float *) pn.w->data, pn.eps };
    }

    void op_rope(int i) {
        rope_batch B{};
        std::vector<int> members;
        add_rope_job(B, members, i);
        if (fuse(FUSE_ROPE)) {
            for (int j = i + 1; j < g_->n_nodes && B.n_jobs < ROPE_MAX_JOBS; j++) {
                const ggml_tensor * m = g_->nodes[j];
                if (done_[j] || std::find(members.begin(), members.end(), j) != members.end() || is_view_op(m->op)) continue;
                // the QK-Norm in front of a later RoPE (held back: nothing runs out of order)
                if (m->op == GGML_OP_RMS_NORM && ready(m->src[0]) && defer_qk_norm(j)) {
                    done_[j] = true;
                    continue;
                }
                if (m->op == GGML_OP_ROPE && m->src[0]->type == GGML_TYPE_F32 && m->type == GGML_TYPE_F32 &&
                    ready(m->src[0]) && ready(m->src[1]) && (!m->src[2] || ready(m->src[2]))) {
                    add_rope_job(B, members, j);
                    continue;
                }
                if (m->op == GGML_OP_CPY && m->src[0]->type == GGML_TYPE_F32 &&
                    (m->type == GGML_TYPE_F16 || m->type == GGML_TYPE_F32) && ready(m->src[0])) {
                    B.job[B.n_jobs++] = rope_job{ tv(m->src[0]), tv(m), nullptr, nullptr, rope_params{}, ggml_nelements(m->src[0]) };
                    members.push_back(j);
                    wrote_.push_back(m);
                    continue;
                }
                break;
            }
        }
        if (defer_rope(B, members)) {
            for (int j : members) done_[j] = true;
            return;
        }
        // a held-back QK-Norm of a rotation's input runs inside the RoPE launch (one wave per row)
        // where its rows fit, otherwise just before it
        for (int j : members) {
            const ggml_tensor * r = g_->nodes[j];
            if (r->op != GGML_OP_ROPE) continue;
            const ggml_tensor * m = r->src[0];
            auto it = pnorm_.find(m);
            if (it == pnorm_.end()) continue;
            const ggml_tensor * x = it->second.x;
            rope_job * J = nullptr;
            for (int k = 0; k < B.n_jobs; k++) if (B.job[k].pos && B.job[k].src.data == (char *) m->data) J = &B.job[k];
            const bool fits = J && fuse(FUSE_NORM) && x->ne[0] == m->ne[0] && x->ne[0] <= 256 && x->nb[0] == sizeof(float) &&
                              x->ne[1] == m->ne[1] && x->ne[2] == m->ne[2] && x->ne[3] == 1 && m->ne[3] == 1 &&
                              J->p.n_dims <= m->ne[0];
            if (!fits) {
                materialize_norm(m);
                continue;
            }
            const qk_norm qn = qk_norm_of(m);
            J->norm_x = qn.x;
            J->norm_nb1 = qn.nb1;
            J->norm_nb2 = qn.nb2;
            J->norm_w = qn.w;
            J->norm_eps = qn.eps;
            J->n = m->ne[1] * m->ne[2];
        }
        // many tokens (prefill): the rotations read one (cos, sin) table per graph instead of
        // forming the same angles for every head of every layer
        for (int k = 0; k < B.n_jobs; k++) {
            rope_job & J = B.job[k];
            const int64_t n_pos = J.src.ne[2];
            if (J.pos && n_pos >= ROPE_TABLE_MIN_TOKENS && J.p.n_dims >= 2) J.cs = rope_table_of(J, n_pos);
        }
        {
            prof_scope ps(this, "rope", 0);
            launch_rope_batch(B, st_);
        }
        for (int j : members) done_[j] = true;
    }

    // A RoPE batch of exactly {Q rotation, K rotation copied into the K cache, V copy into the V
    // cache} whose rotated Q is read only by a decode attention over those caches, with the new
    // rows at that attention's last n_q positions: it runs inside the attention's scores kernel
    // (attn_launch.rope) instead of in a launch of its own.
    struct pending_rope { int anchor = -1; rope_job q, k, v; qk_norm qn, kn; };
    // the (cos, sin) table of the graph's folded RoPE (written by the first attention that uses it)
    float2 * cs_tab_ = nullptr;
    const int32_t * cs_pos_ = nullptr;
    const float * cs_ff_ = nullptr;
    int cs_n_ = 0;
    rope_params cs_p_{};
    pending_rope prope_;
    // the (cos, sin) table of a multi-token RoPE (prefill), formed once per graph for the rotations of
    // the same positions and parameters (Q and K of every layer)
    struct rope_table { float2 * tab; const int32_t * pos; const float * ff; int64_t n; rope_params p; };
    std::vector<rope_table> rope_tabs_;
    const float2 * rope_table_of(const rope_job & J, int64_t n_pos) {
        for (const rope_table & t : rope_tabs_) {
            if (t.pos == J.pos && t.ff == J.ff && t.n == n_pos && memcmp(&t.p, &J.p, sizeof(rope_params)) == 0) return t.tab;
        }
        float2 * tab = (float2 *) c_.scratch.alloc((size_t) n_pos * (J.p.n_dims / 2) * sizeof(float2));
        {
            prof_scope ps(this, "rope_table", 0);
            launch_rope_table(J.pos, n_pos, J.p, J.ff, tab, st_);
        }
        rope_tabs_.push_back(rope_table{ tab, J.pos, J.ff, n_pos, J.p });
        return tab;
    }

    bool defer_rope(const rope_batch & B, const std::vector<int> & members) {
        if (!fuse(FUSE_ATTN) || B.n_jobs != 3 || members.size() != 4) return false;
        int qi = -1, kc = -1, vc = -1;
        for (int j : members) {
            const ggml_tensor * m = g_->nodes[j];
            if (m->op == GGML_OP_ROPE) {
                const int u = sole_user(j);
                const bool copied = u >= 0 && g_->nodes[u]->op == GGML_OP_CPY &&
                                    std::find(members.begin(), members.end(), u) != members.end();
                if (!copied) qi = j;
            } else if (m->op == GGML_OP_CPY) {
                if (m->src[0]->op == GGML_OP_ROPE) kc = j;
                else vc = j;
            }
        }
        if (qi < 0 || kc < 0 || vc < 0) return false;
        int jq = -1, jk = -1, jv = -1;
        for (int k = 0; k < 3; k++) {
            const rope_job & J = B.job[k];
            if (J.dst.data == g_->nodes[qi]->data && J.pos) jq = k;
            else if (J.dst.data == g_->nodes[kc]->data && J.pos) jk = k;
            else if (J.dst.data == g_->nodes[vc]->data && !J.pos) jv = k;
        }
        if (jq < 0 || jk < 0 || jv < 0) return false;
        // Q and K rotate with the same positions, frequency factors and parameters (one table of
        // rotation pairs serves both), over at most the head dimension
        const rope_job & q = B.job[jq], & k = B.job[jk];
        if (q.pos != k.pos || q.ff != k.ff || memcmp(&q.p, &k.p, sizeof(rope_params)) != 0 || q.p.n_dims > q.src.ne[0]) return false;
        // the sources are f32 rows of contiguous elements (read as rows by the scores kernel)
        const rope_job & v = B.job[jv];
        if (q.src.type != GGML_TYPE_F32 || k.src.type != GGML_TYPE_F32 || v.src.type != GGML_TYPE_F32 ||
            q.src.nb[0] != 4 || k.src.nb[0] != 4 || v.src.nb[0] != 4) return false;
        // rotated Q -> permute -> the attention anchor (and nothing else)
        const int p = sole_user(qi);
        if (p < 0 || g_->nodes[p]->op != GGML_OP_PERMUTE) return false;
        const int a = sole_user(p);
        auto it = attn_.find(a);
        if (a < 0 || it == attn_.end()) return false;
        const attn_match & M = it->second;
        const ggml_tensor * kp = M.kp, * vp = M.vp, * qp = M.qp;
        const ggml_tensor * kn = g_->nodes[kc], * vn = g_->nodes[vc];
        const int64_t hd = kp->ne[0], n_kv = kp->ne[1], n_head_kv = kp->ne[2], n_q = qp->ne[1], n_head = qp->ne[2];
        if (qp != g_->nodes[p] || n_q > 4 || n_kv < n_q || kn->type != GGML_TYPE_F16 || vn->type != GGML_TYPE_F16) return false;
        const int64_t shape_q[3] = { hd, n_head, n_q }, shape_kv[3] = { hd, n_head_kv, n_q };
        for (int d = 0; d < 3; d++) {
            if (B.job[jq].src.ne[d] != shape_q[d] || B.job[jk].src.ne[d] != shape_kv[d] ||
                B.job[jv].src.ne[d] != shape_kv[d] || kn->ne[d] != shape_kv[d] || vn->ne[d] != shape_kv[d]) return false;
        }
        // the new rows are the attention's last n_q positions of the same caches
        if ((const char *) kn->data != (const char *) kp->data + (n_kv - n_q) * kp->nb[1] ||
            kn->nb[1] != kp->nb[2] || kn->nb[2] != kp->nb[1] || kn->nb[0] != 2) return false;
        if ((const char *) vn->data != (const char *) vp->data + (n_kv - n_q) * vp->nb[0] ||
            vn->nb[1] != vp->nb[2] || vn->nb[2] != vp->nb[0] || vn->nb[0] != 2) return false;
        // held-back QK-Norms of the rotated Q and K (their rows: hd contiguous floats)
        const ggml_tensor * qsrc = g_->nodes[qi]->src[0], * ksrc = g_->nodes[kc]->src[0]->src[0];
        for (const ggml_tensor * src : { qsrc, ksrc }) {
            auto it = pnorm_.find(src);
            if (it != pnorm_.end() && (it->second.x->ne[0] != hd || it->second.x->nb[0] != sizeof(float) ||
                                       ggml_nrows(it->second.x) > 4 * 64)) return false;
        }
        prope_ = pending_rope{ a, B.job[jq], B.job[jk], B.job[jv], qk_norm_of(qsrc), qk_norm_of(ksrc) };
        wrote_.push_back(g_->nodes[kc]);
        wrote_.push_back(g_->nodes[vc]);
        return true;
    }

    // the lowest node index that reads node u's data, directly or through views (INT_MAX: none)
    int first_reader(int u) const {
        int first = INT_MAX;
        for (int j : users_[u]) {
            const ggml_tensor * t = g_->nodes[j];
            first = std::min(first, is_view_op(t->op) ? first_reader(j) : j);
        }
        return first;
    }

    // the highest node index that reads node u's data, directly or through views (INT_MAX: an
    // output, live to the end of the graph)
    int last_reader(int u) const {
        if (is_output(u)) return INT_MAX;
        int last = -1;
        for (int j : users_[u]) {
            const ggml_tensor * t = g_->nodes[j];
            last = std::max(last, is_view_op(t->op) ? std::max(j, last_reader(j)) : j);
        }
        return last;
    }

    // The MoE FFN norm: rms_norm -> mul(w) whose first reader in node order is the F32 router
    // mul_mat (build_moe_ffn's ffn_gate_inp product). Nothing is launched here: the router launch
    // normalizes each column itself and writes the mul's output for the later readers (the expert
    // GEMVs), so the norm costs no launch of its own.
    bool defer_router_norm(int i, int u, float eps) {
        if (!fuse(FUSE_ROUTE) || is_output(u)) return false;
        const ggml_tensor * n = g_->nodes[i], * m = g_->nodes[u];
        const ggml_tensor * x = n->src[0];
        const int r = first_reader(u);
        if (r == INT_MAX) return false;
        const ggml_tensor * rn = g_->nodes[r];
        if (rn->op != GGML_OP_MUL_MAT || rn->src[1] != m || !is_2d_contig(rn) || !is_2d_contig(m)) return false;
        if (!mul_mat_rows_norm_supported(tv(rn->src[0]), x->ne[0]) || x->ne[2] != 1 || x->ne[3] != 1 || x->nb[0] != 4 ||
            x->nb[1] % 4) {
            return false;
        }
        // the router launch reads x at node r, later than the allocator planned for, and writes m:
        // x must be disjoint from m and stay live up to r (read again at or after r, or not a node
        // of this graph), else the allocator may have placed m or a node before r over it
        const char * xb = (const char *) x->data, * mb = (const char *) m->data;
        if (xb < mb + ggml_nbytes(m) && mb < xb + ggml_nbytes(x)) return false;
        const int xi = node_index(x->view_src ? x->view_src : x);
        if (xi >= 0 && last_reader(xi) < r) return false;
        router_norm_[r] = router_norm{ i, u, eps };
        done_[u] = true;
        return true;
    }

    // rms_norm, fused with a following weight multiply (and activation quantization) when possible
    void op_rms_norm(int i) {
        ggml_tensor * n = g_->nodes[i];
        float eps;
        memcpy(&eps, n->op_params, 4);
        const ggml_tensor * x = n->src[0];
        const bool rows_ok = x->type == GGML_TYPE_F32 && ggml_is_contiguous(x) && ggml_is_contiguous(n) &&
                             x->ne[0] <= RMS_NORM_MAX_ROW;
        if (fuse(FUSE_NORM) && rows_ok) {
            const int u = sole_user(i);
            if (u >= 0) {
                ggml_tensor * m = g_->nodes[u];
                const ggml_tensor * w = m->src[1];
                if (m->op == GGML_OP_MUL && m->src[0] == n && w->type == GGML_TYPE_F32 && ggml_nrows(w) == 1 &&
                    w->ne[0] == x->ne[0] && ggml_is_contiguous(w) && ggml_is_contiguous(m)) {
                    const int64_t N = x->ne[0], rows = ggml_nrows(x);
                    if (defer_qk_norm(i)) return;
                    if (defer_router_norm(i, u, eps)) return;
                    if (m->ne[1] == rows && norm_deferrable(u, N) && ((uintptr_t) x->data | (uintptr_t) w->data) % 16 == 0) {
                        const gemv_norm nz{ (const float *) x->data, N, (const float *) w->data, eps, 1 };
                        done_[u] = true;
                        if (max_consumer_rows(u) <= GEMV_PROLOGUE_MAX_ROWS && !gemm_consumer(u) && (rows == 1 || !fuse(FUSE_MC))) {
                            norm_[m] = nz;      // every consumer workgroup normalizes for itself
                            return;
                        }
                        // a very wide consumer (the LM head) or a GEMM: normalize and quantize once
                        const int wtype = gemv_only_consumers(u);
                        const int kind = dot_kind(wtype);
                        act_entry e = alloc_act(kind, N, rows);
                        gemv_launch L{};
                        L.type = wtype;
                        L.K = (int) N;
                        L.ncols = (int) rows;
                        L.norm = nz;
                        {
                            prof_scope ps(this, "act_quant", (double) (N * rows * 4 + N * 4));
                            launch_act_quant(L, e.q8, e.q8k, st_);
                        }
                        act_[m] = e;
                        return;
                    }
                    const int kind = m->ne[1] == rows ? wanted_act_kind(u) : 0;
                    act_entry e{};
                    const bool q = (kind == 1 && N % 32 == 0) || (kind == 2 && N % 256 == 0);
                    if (q) e = alloc_act(kind, N, rows);
                    prof_scope ps(this, "rms_norm_mul", (double) (N * rows * 8 + N * 4));
                    launch_rms_norm((const float *) x->data, N, (const float *) w->data, (float *) m->data, N, N, rows, eps,
                                    q && kind == 1 ? &e.q8 : nullptr, q && kind == 2 ? &e.q8k : nullptr, st_);
                    if (q) act_[m] = e;
                    done_[u] = true;
                    wrote_.push_back(m);
                    return;
                }
            }
        }
        wrote_.push_back(n);
        prof_scope ps(this, "rms_norm", 0);
        if (rows_ok) {
            launch_rms_norm((const float *) x->data, x->ne[0], nullptr, (float *) n->data, n->ne[0], x->ne[0], ggml_nrows(x), eps,
                            nullptr, nullptr, st_);
        } else {
            launch_rms_norm_strided(tv(x), tv(n), eps, st_);
        }
    }

    bool gemv_capable(const ggml_tensor * mm) const {
        const ggml_tensor * w = mm->src[0];
        const ggml_tensor * x = mm->src[1];
        if (!dot_kind(w->type)) return false;
        if (w->ne[0] % (is_kquant(w->type) ? 256 : 32)) return false;
        if (x->type != GGML_TYPE_F32 || x->nb[0] != sizeof(float)) return false;
        if (mm->op == GGML_OP_MUL_MAT_ID) {
            // experts [K, N, n_expert] stored contiguously; activation [K, x_cols, n_tok] with evenly
            // strided rows; output [N, n_slots, n_tok] contiguous
            const ggml_tensor * ids = mm->src[2];
            return ggml_is_contiguous(w) && w->ne[3] == 1 && x->ne[3] == 1 && x->nb[2] == x->nb[1] * x->ne[1] &&
                   ids->type == GGML_TYPE_I32 && ids->nb[0] == sizeof(int32_t) && ggml_is_contiguous(mm);
        }
        if (!is_2d_contig(w)) return false;
        if (x->ne[2] != 1 || x->ne[3] != 1) return false;
        return is_2d_contig(mm);
    }

    // a quantized mul_mat over a prefill-width batch: the int8-MFMA GEMM (same floats as the GEMV)
    bool gemm_route(const ggml_tensor * mm) const {
        const int64_t cols = mm->src[1]->ne[1];
        const bool wide = cols >= GEMM_MIN_COLS || (cols >= GEMM_WIDE_MIN_COLS && mm->src[0]->ne[1] >= GEMM_WIDE_MIN_ROWS);
        return mm->op == GGML_OP_MUL_MAT && wide && gemv_capable(mm) &&
               gemm_supported(mm->src[0]->type, mm->src[0]->ne[0], mm->src[0]->ne[1]) &&
               (mm->nb[1] / sizeof(float)) % 4 == 0 && ((uintptr_t) mm->data) % 16 == 0 &&
               (is_repacked(mm->src[0]->type) || ((uintptr_t) mm->src[0]->data) % 16 == 0);
    }
    bool gemm_consumer(int u) const {
        for (int j : users_[u]) if (gemm_route(g_->nodes[j])) return true;
        return false;
    }

    void op_gemm(int i) {
        ggml_tensor * n = g_->nodes[i];
        const ggml_tensor * w = n->src[0];
        const ggml_tensor * x = n->src[1];
        const int kind = dot_kind(w->type);
        const act_entry * xa = ensure_act(x, kind);
        gemm_launch G{};
        G.type = w->type;
        G.K = w->ne[0];
        G.n_rows = w->ne[1];
        G.ncols = x->ne[1];
        if (kind == 2) {
            if (w->type == GGML_TYPE_Q6_K) {
                const planes p = planes_of(w);
                G.w = p.qs + p.first_block * 128;
                G.wqh = p.qh + p.first_block * 64;
                G.wsc = p.sc + p.first_block * 16;
                G.wd = p.d + p.first_block;
            } else {
                G.w = (const uint8_t *) w->data;
            }
            G.xq = xa->q8k.qs;
            G.xd = xa->q8k.d;
            G.xbs = xa->q8k.bsums;
        } else {
            const planes p = planes_of(w);
            G.w = p.qs + p.first_block * qs_bytes_of(w->type);
            G.wd = p.d + p.first_block;
            G.xq = xa->q8.qs;
            G.xd = xa->q8.d;
        }
        G.y = (float *) n->data;
        G.y_stride = (int64_t) (n->nb[1] / sizeof(float));
        const double act_bytes = kind == 2 ? 1.0 + 4.0 / 256 + 2.0 / 16 : 1.0 + 4.0 / 32;
        double bytes = (double) ggml_nbytes(w) + (double) (G.K * G.ncols) * act_bytes + (double) (G.n_rows * G.ncols * 4);
        ggml_tensor * written = n;
        const int u = fuse(FUSE_ADD) ? sole_user(i) : -1;
        if (u >= 0) {
            ggml_tensor * an = g_->nodes[u];
            if (an->op == GGML_OP_ADD && an->src[0] == n && an->src[1]->type == GGML_TYPE_F32 &&
                ggml_are_same_shape(an->src[1], n) && is_2d_contig(an->src[1]) && is_2d_contig(an) &&
                (((uintptr_t) an->data | (uintptr_t) an->src[1]->data) % 16) == 0 &&
                (an->nb[1] / sizeof(float)) % 4 == 0 && (an->src[1]->nb[1] / sizeof(float)) % 4 == 0) {
                G.y = (float *) an->data;
                G.y_stride = (int64_t) (an->nb[1] / sizeof(float));
                G.add = (const float *) an->src[1]->data;
                G.add_stride = (int64_t) (an->src[1]->nb[1] / sizeof(float));
                bytes += (double) (G.n_rows * G.ncols * 4);
                done_[u] = true;
                written = an;
            }
        }
        {
            // named with the workgroup tile, e.g. gemm_q8_0_2x4x2
            const std::string pname = std::string("gemm_") + ggml_type_name(w->type) + "_" + gemm_tile_name(G);
            prof_scope ps(this, pname.c_str(), bytes);
            launch_gemm(G, st_);
        }
        wrote_.push_back(written);
        done_[i] = true;
    }

    void op_mul_mat(int i) {
        ggml_tensor * n = g_->nodes[i];
        auto at = attn_.find(i);
        if (at != attn_.end()) { run_attention(at->second); return; }
        if (gemm_route(n)) { op_gemm(i); return; }
        if (gemv_capable(n)) { op_gemv(i); return; }
        if (ggml_is_quantized(n->src[0]->type)) {
            HIP_ABORT("mul_mat '%s': quantized %s weights with this layout are not supported", n->name, ggml_type_name(n->src[0]->type));
        }
        if (n->src[1]->type != GGML_TYPE_F32 || n->src[0]->nb[0] != ggml_type_size(n->src[0]->type)) {
            HIP_ABORT("mul_mat '%s': unsupported operand layout", n->name);
        }
        auto rn = router_norm_.find(i);
        if (rn != router_norm_.end()) {
            const ggml_tensor * x = g_->nodes[rn->second.norm]->src[0];
            ggml_tensor * m = g_->nodes[rn->second.mul];
            const ggml_tensor * nw = m->src[1];
            wrote_.push_back(m);
            wrote_.push_back(n);
            // the norm's other readers all K-quant GEMVs (the MoE experts): its Q8_K form too, so
            // that they quantize nothing
            // (directly or through a contiguous reshape that keeps the row length: build_moe_ffn's
            // [n_embd, 1, n_tokens] view)
            q8k_act q8k{};
            if (fuse(FUSE_ACTQ) && m->ne[0] % 256 == 0 && is_2d_contig(m)) {
                bool kq = false, other = false;
                std::vector<const ggml_tensor *> readers = { m };
                auto kq_reader = [&](const ggml_tensor * un, const ggml_tensor * src) {
                    return (un->op == GGML_OP_MUL_MAT || un->op == GGML_OP_MUL_MAT_ID) && un->src[1] == src &&
                           un->src[0] != src && dot_kind(un->src[0]->type) == 2;
                };
                for (int j : users_[rn->second.mul]) {
                    const ggml_tensor * un = g_->nodes[j];
                    if (j == i) continue;
                    if (kq_reader(un, m)) {
                        kq = true;
                    } else if (un->op == GGML_OP_RESHAPE && un->src[0] == m && un->data == m->data && ggml_is_contiguous(un) &&
                               un->ne[0] == m->ne[0] && !users_[j].empty()) {
                        for (int k : users_[j]) {
                            if (kq_reader(g_->nodes[k], un)) kq = true;
                            else other = true;
                        }
                        readers.push_back(un);
                    } else {
                        other = true;
                    }
                }
                if (kq && !other) {
                    act_entry e = alloc_act(2, m->ne[0], m->ne[1]);
                    q8k = e.q8k;
                    for (const ggml_tensor * r : readers) act_[r] = e;
                }
            }
            prof_scope ps(this, "router_norm", (double) (ggml_nbytes(n->src[0]) + 2 * ggml_nbytes(x) + ggml_nbytes(n)));
            launch_mul_mat_rows_norm(tv(n->src[0]), (const float *) x->data, (int64_t) (x->nb[1] / 4), (const float *) nw->data,
                                     rn->second.eps, (float *) m->data, (int64_t) (m->nb[1] / 4), tv(n), x->ne[1], q8k, st_);
            return;
        }
        wrote_.push_back(n);
        prof_scope ps(this, "mul_mat_generic", (double) (ggml_nbytes(n->src[0]) + ggml_nbytes(n->src[1]) + ggml_nbytes(n)));
        launch_mul_mat_generic(tv(n->src[0]), tv(n->src[1]), tv(n), st_);
    }

    // Columns per grouped workgroup: about the columns an active expert gets with uniform routing
    // (1 - (1 - k/E)^T of the experts are active), as a power of two in [2, 16]
    static int moe_cols_per_item(int n_slots, int n_tok, int n_experts) {
        const double active = n_experts * (1.0 - std::pow(1.0 - std::min(1.0, (double) n_slots / n_experts), (double) n_tok));
        const double avg = (double) n_slots * n_tok / std::max(1.0, active);
        int nc = 2;
        while (nc < GEMV_MC_MAX_COLS && nc < avg) nc *= 2;
        return nc;
    }

    // distinct values in [0, n) of an I32 ids tensor [slots, tokens] (copied back synchronously)
    int64_t distinct_ids(const ggml_tensor * ids, int64_t n) {
        const int64_t ns = ids->ne[0], nt = ids->ne[1];
        std::vector<int32_t> h((size_t) (ns * nt));
        HIP_CHECK(hipMemcpy2DAsync(h.data(), (size_t) ns * 4, ids->data, ids->nb[1], (size_t) ns * 4, (size_t) nt,
                                   hipMemcpyDeviceToHost, st_));
        HIP_CHECK(hipStreamSynchronize(st_));
        std::vector<char> seen((size_t) n, 0);
        int64_t k = 0;
        for (int32_t v : h) {
            if (v >= 0 && v < n && !seen[(size_t) v]) { seen[(size_t) v] = 1; k++; }
        }
        return k;
    }

    // The columns of a mul_mat_id grouped by expert (once per ids tensor and graph compute)
    std::unordered_map<const ggml_tensor *, expert_groups> groups_;
    const expert_groups & expert_groups_of(const ggml_tensor * ids, int n_experts) {
        auto it = groups_.find(ids);
        if (it != groups_.end()) return it->second;
        const int n_slots = (int) ids->ne[0], n_tok = (int) ids->ne[1], ncol = n_slots * n_tok;
        expert_groups g{};
        g.nc = moe_cols_per_item(n_slots, n_tok, n_experts);
        g.max_items = std::min(n_experts, ncol) + (ncol + g.nc - 1) / g.nc;
        g.count = (int32_t *) c_.scratch.alloc((size_t) n_experts * sizeof(int32_t));
        g.offset = (int32_t *) c_.scratch.alloc((size_t) n_experts * sizeof(int32_t));
        g.cols = (int32_t *) c_.scratch.alloc((size_t) ncol * sizeof(int32_t));
        g.items = (int32_t *) c_.scratch.alloc((size_t) g.max_items * 3 * sizeof(int32_t));
        g.n_items = (int32_t *) c_.scratch.alloc(sizeof(int32_t));
        {
            prof_scope ps(this, "moe_group", 0);
            launch_moe_group((const int32_t *) ids->data, (int64_t) (ids->nb[1] / sizeof(int32_t)), n_slots, n_tok, n_experts, g, st_);
        }
        return groups_[ids] = g;
    }

    // Whether the GEMVs of a group read activation x (f32, not yet quantized) straight from memory,
    // quantizing it in their prologue, rather than after a quantization launch of its own: for
    // launches whose rows (per column) are few enough that redoing it per workgroup stays cheap.
    bool quantize_in_prologue(const ggml_tensor * x, int wtype, const std::vector<int> & group, bool by_id) const {
        if (!fuse(FUSE_ACTQ) || x->type != GGML_TYPE_F32 || x->nb[0] != sizeof(float) || x->ne[3] != 1) return false;
        if (((uintptr_t) x->data) % 16 || x->nb[1] % 16 || x->ne[0] > gemv_prologue_max_k(wtype, false)) return false;
        // columns evenly strided (mul_mat_id reads column t * ne[1] + slot)
        if (x->ne[2] > 1 && x->nb[2] != x->nb[1] * x->ne[1]) return false;
        if (!by_id && x->ne[2] > 1) return false;
        int64_t rows = 0;
        for (int j : group) rows += g_->nodes[j]->src[0]->ne[1];
        return rows <= GEMV_PROLOGUE_MAX_ROWS;
    }

    // quantized GEMV for node i, grouped with the other pending mul_mats that read the same input
    void op_gemv(int i) {
        ggml_tensor * n = g_->nodes[i];
        const ggml_tensor * x = n->src[1];
        const int wtype = n->src[0]->type;
        const bool by_id = n->op == GGML_OP_MUL_MAT_ID;
        const ggml_tensor * ids = by_id ? n->src[2] : nullptr;
        const int64_t K = n->src[0]->ne[0];
        const int64_t ncols = by_id ? ids->ne[0] * ids->ne[1] : x->ne[1];   // launch columns
        std::vector<int> group = { i };
        if (fuse(FUSE_GROUP)) {
            const int xi = node_index(x);
            std::vector<int> others;
            if (xi < 0) {
                for (int j = i + 1; j < g_->n_nodes; j++) {
                    const ggml_tensor * m = g_->nodes[j];
                    if (m->op == n->op && m->src[1] == x) others.push_back(j);
                }
            } else {
                for (int j : users_[xi]) if (j != i) others.push_back(j);
            }
            for (int j : others) {
                const ggml_tensor * m = g_->nodes[j];
                if (done_[j] || m->op != n->op || m->src[1] != x || (by_id && m->src[2] != ids)) continue;
                if (attn_.count(j)) continue;
                if (m->src[0]->type != wtype || m->src[0]->ne[0] != K || !gemv_capable(m)) continue;
                if ((int) group.size() == GEMV_MAX_MATS) break;
                group.push_back(j);
            }
        }

        // SwiGLU pair inside the group: gate -> silu -> mul(silu, up)
        int gate = -1, up = -1, mulnode = -1;
        if (fuse(FUSE_SWIGLU) && group.size() >= 2 && K <= gemv_swiglu_max_k(wtype)) {
            for (int a : group) {
                const int s = sole_user(a);
                if (s < 0) continue;
                const ggml_tensor * sn = g_->nodes[s];
                if (sn->op != GGML_OP_UNARY || sn->op_params[0] != GGML_UNARY_OP_SILU) continue;
                const int m = sole_user(s);
                if (m < 0) continue;
                const ggml_tensor * mn = g_->nodes[m];
                if (mn->op != GGML_OP_MUL || mn->src[0] != sn) continue;
                const int b = node_index(mn->src[1]);
                if (b < 0 || sole_user(b) != m || std::find(group.begin(), group.end(), b) == group.end()) continue;
                if (!ggml_are_same_shape(g_->nodes[a], g_->nodes[b]) || !(by_id ? ggml_is_contiguous(mn) : is_2d_contig(mn))) continue;
                gate = a; up = b; mulnode = m;
                break;
            }
        }

        const int kind = dot_kind(wtype);
        // several columns (tokens) per workgroup: the activation is quantized once, up front
        const int64_t n_tok = by_id ? ids->ne[1] : ncols;
        const int mc_nc = by_id ? moe_cols_per_item((int) ids->ne[0], (int) n_tok, (int) n->src[0]->ne[2]) : 0;
        const bool mc = fuse(FUSE_MC) && n_tok >= 2 && gemv_mc_fits(wtype, (int) K, false, mc_nc) &&
                        (gate < 0 || gemv_mc_fits(wtype, (int) K, true, mc_nc));
        const auto nz = norm_.find(x);
        gemv_norm pro{};
        const act_entry * xa = nullptr;
        if (mc) {
            if (act_.count(x) && act_.at(x).kind == kind) {
                xa = &act_.at(x);
            } else if (nz != norm_.end() && K <= act_quant_max_k(wtype, nz->second.rms != 0)) {
                act_entry e = alloc_act(kind, K, ggml_nrows(x));
                gemv_launch Q{};
                Q.type = wtype;
                Q.K = (int) K;
                Q.ncols = (int) ggml_nrows(x);
                Q.norm = nz->second;
                {
                    prof_scope ps(this, "act_quant", (double) (K * ggml_nrows(x) * 4));
                    launch_act_quant(Q, e.q8, e.q8k, st_);
                }
                act_[x] = e;
                xa = &act_[x];
            } else {
                if (nz != norm_.end()) HIP_ABORT("mul_mat '%s': normalized input too long to quantize", n->name);
                xa = ensure_act(x, kind);
            }
        } else if (nz != norm_.end()) {
            pro = nz->second;
        } else if (act_.count(x) && act_.at(x).kind == kind) {
            xa = &act_.at(x);
        } else if (quantize_in_prologue(x, wtype, group, by_id)) {
            // an f32 activation nobody quantized: every workgroup quantizes it in its prologue
            pro = gemv_norm{ (const float *) x->data, (int64_t) (x->nb[1] / sizeof(float)), nullptr, 0.0f, 0 };
        } else {
            xa = ensure_act(x, kind);
        }

        // profiled steps only: the ids back on the host, to count the distinct experts a
        // mul_mat_id reads (a synchronization, never inside a timed region)
        int64_t n_unique_experts = -1;
        auto fill_mat = [&](gemv_mat & gm, int j, double & bytes, bool epilogue) {
            ggml_tensor * mm = g_->nodes[j];
            const ggml_tensor * w = mm->src[0];
            gm.wqh = nullptr;
            gm.wsc = nullptr;
            if (is_repacked(w->type)) {
                const planes p = planes_of(w);
                gm.w = p.qs + p.first_block * qs_bytes_of(w->type);
                gm.wd = p.d + p.first_block;
                if (w->type == GGML_TYPE_Q6_K) {
                    gm.wqh = p.qh + p.first_block * 64;
                    gm.wsc = p.sc + p.first_block * 16;
                }
            } else {
                gm.w = (const uint8_t *) w->data;
                gm.wd = nullptr;
            }
            gm.n_rows = (int32_t) w->ne[1];
            gm.y = (float *) mm->data;
            gm.y_stride = (int64_t) (mm->nb[1] / sizeof(float));
            gm.add = nullptr;
            gm.add_stride = 0;
            // the weights one launch must read: every row, or the rows of the selected experts
            // (each distinct one once: counted from the ids in profiled steps, else bounded by the
            // columns)
            const double wbytes = !by_id ? (double) ggml_nbytes(w)
                                  : n_unique_experts >= 0 ? (double) n_unique_experts * (double) w->nb[2]
                                  : std::min((double) ggml_nbytes(w), (double) ncols * (double) w->nb[2]);
            bytes += wbytes + (double) (w->ne[1] * ncols * 4);
            const ggml_tensor * written = mm;
            // residual add epilogue
            const int u = (epilogue && fuse(FUSE_ADD)) ? sole_user(j) : -1;
            if (u >= 0) {
                ggml_tensor * an = g_->nodes[u];
                if (an->op == GGML_OP_ADD && an->src[0] == mm && an->src[1]->type == GGML_TYPE_F32 &&
                    ggml_are_same_shape(an->src[1], mm) && is_2d_contig(an->src[1]) && is_2d_contig(an)) {
                    gm.y = (float *) an->data;
                    gm.y_stride = (int64_t) (an->nb[1] / sizeof(float));
                    gm.add = (const float *) an->src[1]->data;
                    gm.add_stride = (int64_t) (an->src[1]->nb[1] / sizeof(float));
                    bytes += (double) (w->ne[1] * ncols * 4);
                    done_[u] = true;
                    written = an;
                }
            }
            if (epilogue) wrote_.push_back(written);
        };

        gemv_launch L{};
        L.type = wtype;
        L.K = (int) K;
        L.ncols = (int) ncols;
        if (!xa) L.norm = pro;
        else if (kind == 1) { L.xq = xa->q8.qs; L.xd = xa->q8.d; L.xs = xa->q8.s; }
        else { L.xq = xa->q8k.qs; L.xd = xa->q8k.d; L.xbs = xa->q8k.bsums; }
        if (by_id) {
            L.ids = (const int32_t *) ids->data;
            L.ids_stride = (int64_t) (ids->nb[1] / sizeof(int32_t));
            L.n_slots = (int) ids->ne[0];
            L.x_cols = (int) x->ne[1];
            L.n_experts = (int) n->src[0]->ne[2];
            L.expert_rows = n->src[0]->ne[1];
        }
        // a one-token routing held back for this launch: run inside the SwiGLU launch when that is
        // the single-column Q4_K kernel, else launched now, before anything reads its ids
        bool route_in = false;
        moe_route route{};
        if (by_id) {
            auto it = pending_route_.find(ids);
            if (it != pending_route_.end()) {
                route = it->second;
                pending_route_.erase(it);
                if (gate >= 0 && !mc && gemv_q4k_enabled()) {
                    gemv_launch P = L;
                    P.n_mats = 2;
                    P.swiglu = true;
                    P.route_logits = route.logits;
                    P.route_w = route.w;
                    P.route_scale = route.scale;
                    route_in = route.n_expert == L.n_experts && route.k == L.n_slots && L.ids == route.ids &&
                               gemv_q4k_supported(P);
                }
                if (!route_in) run_route(route);
            }
        }
        if (by_id && c_.timing && !route_in) n_unique_experts = distinct_ids(ids, n->src[0]->ne[2]);
        const double x_bytes = (double) (K * ggml_nrows(x) * 4) + (xa ? 0.0 : (double) (K * 4));
        // one column per workgroup, or several (mul_mat_id: the tokens routed to each expert)
        const expert_groups * G = mc && by_id ? &expert_groups_of(ids, (int) n->src[0]->ne[2]) : nullptr;
        auto run = [&](const gemv_launch & X) {
            // GGML_HIP_NO_MFMA_GEMV: the multi-column GEMV for every such launch (comparisons)
            static const bool no_mfma = getenv("GGML_HIP_NO_MFMA_GEMV") != nullptr;
            if (mc && !G && !no_mfma && gemv_mfma_supported(X)) launch_gemv_mfma(X, st_);
            else if (mc) launch_gemv_mc(X, G, G ? (int) n_tok : X.ncols, st_);
            else launch_gemv(X, st_);
        };

        if (gate >= 0) {
            // SwiGLU launch for (gate, up); the rest of the group goes in a second launch
            gemv_launch S = L;
            S.n_mats = 2;
            S.swiglu = true;
            double sb = x_bytes;
            fill_mat(S.m[0], gate, sb, false);
            fill_mat(S.m[1], up, sb, false);
            ggml_tensor * mn = g_->nodes[mulnode];
            S.m[0].y = (float *) mn->data;
            S.m[0].y_stride = (int64_t) (mn->nb[1] / sizeof(float));
            S.m[0].add = nullptr;
            sb -= (double) (g_->nodes[gate]->ne[0] * ncols * 4); // gate/up outputs are not written, act is
            // the GEMVs reading act (the down projection): Q8_0 consumers read it pre-quantized, the
            // launch writing its blocks; others quantize it in their prologue
            const int dtype = fuse(FUSE_ACTQ) && !mc ? gemv_only_consumers(mulnode) : -1;
            if (dtype >= 0 && dot_kind(dtype) == 1 && gemv_q_supported(S) && K <= GEMV_SWIGLU_QOUT_MAX_K && mn->ne[0] % 32 == 0 &&
                is_2d_contig(mn)) {
                act_entry e = alloc_act(1, mn->ne[0], ggml_nrows(mn));
                S.out_q = e.q8;
                act_[mn] = e;
            } else if (dtype >= 0 && mn->ne[0] <= gemv_prologue_max_k(dtype, false) && ((uintptr_t) mn->data) % 16 == 0) {
                norm_[mn] = gemv_norm{ (const float *) mn->data, (int64_t) (mn->nb[1] / sizeof(float)), nullptr, 0.0f, 0 };
            }
            if (route_in) {
                S.route_logits = route.logits;
                S.route_w = route.w;
                S.route_scale = route.scale;
                sb += (double) (route.n_expert * 4 + route.k * 8);
            }
            {
                prof_scope ps(this, route_in ? "gemv_q4_K_swiglu_route" : gemv_prof_name(wtype, true), sb);
                if (route_in) launch_gemv(S, st_);
                else run(S);
                if (route_in && c_.timing) {
                    // the experts this launch read, known once it ran (a synchronization; profiled
                    // steps only)
                    n_unique_experts = distinct_ids(ids, n->src[0]->ne[2]);
                    gemv_launch T = S;
                    double tb = x_bytes + (double) (route.n_expert * 4 + route.k * 8);
                    fill_mat(T.m[0], gate, tb, false);
                    fill_mat(T.m[1], up, tb, false);
                    ps.bytes = tb - (double) (g_->nodes[gate]->ne[0] * ncols * 4);
                }
            }
            wrote_.push_back(mn);
            done_[gate] = done_[up] = done_[mulnode] = true;
            done_[sole_user(gate)] = true; // the silu node
            std::vector<int> rest;
            for (int j : group) if (j != gate && j != up) rest.push_back(j);
            group = rest;
            if (group.empty()) return;
        }

        double bytes = x_bytes;
        L.n_mats = (int) group.size();
        for (size_t k = 0; k < group.size(); k++) fill_mat(L.m[k], group[k], bytes, true);
        {
            prof_scope ps(this, gemv_prof_name(wtype, false), bytes);
            run(L);
        }
        for (int j : group) done_[j] = true;
    }

    // silu(gate) -> mul(., up) on f32 2-D views (prefill: the fused gate/up projection's halves, or
    // separate gate and up projections) ==> one element-wise kernel, which also writes the Q8_0 /
    // Q8_K activation its quantized consumers read
    static bool disjoint_or_same(const ggml_tensor * a, const ggml_tensor * b) {
        const uint8_t * a0 = (const uint8_t *) a->data, * b0 = (const uint8_t *) b->data;
        return a0 == b0 || a0 + ggml_nbytes(a) <= b0 || b0 + ggml_nbytes(b) <= a0;
    }
    bool op_swiglu(int i) {
        ggml_tensor * sn = g_->nodes[i];
        if (sn->op_params[0] != GGML_UNARY_OP_SILU) return false;
        const int mj = sole_user(i);
        if (mj < 0) return false;
        ggml_tensor * mn = g_->nodes[mj];
        const ggml_tensor * gt = sn->src[0], * up = mn->src[1];
        if (mn->op != GGML_OP_MUL || mn->src[0] != sn || !ggml_are_same_shape(gt, mn) || !ggml_are_same_shape(up, mn)) return false;
        for (const ggml_tensor * t : { gt, up, (const ggml_tensor *) mn }) {
            if (t->type != GGML_TYPE_F32 || t->nb[0] != sizeof(float) || t->ne[2] != 1 || t->ne[3] != 1) return false;
        }
        // the kernel reads gate[i] and up[i] before writing out[i]: the output may sit exactly on
        // either input, never across one (gate is not an input of the mul, so the allocator may
        // have reused its memory for the output)
        if (!disjoint_or_same(mn, gt) || !disjoint_or_same(mn, up)) return false;
        if (!ready(up)) {
            // separate projections: up comes after the silu. Hold the silu back (nothing launched)
            // when the nodes before the mul are only the up projection on the prefill GEMM (no
            // fused writes elsewhere) and views, and the projection does not write over the gate.
            for (int k = i + 1; k < mj; k++) {
                const ggml_tensor * t = g_->nodes[k];
                if (done_[k] || is_view_op(t->op)) continue;
                if (t != up || !gemm_route(t) || sole_user(k) != mj || !disjoint_or_same(t, gt) || t->data == gt->data) return false;
            }
            silu_of_[mj] = i;
            return true;
        }
        run_swiglu(i, mj);
        return true;
    }
    void run_swiglu(int i, int mj) {
        const ggml_tensor * gt = g_->nodes[i]->src[0];
        ggml_tensor * mn = g_->nodes[mj];
        const ggml_tensor * up = mn->src[1];
        const int64_t K = mn->ne[0], ncols = mn->ne[1];
        const int want = is_2d_contig(mn) ? wanted_act_kind(mj) : 0;
        const int kind = (want == 1 && K % 32 == 0) || (want == 2 && K % 256 == 0) ? want : 0;
        act_entry e{};
        if (kind) e = alloc_act(kind, K, ncols);
        {
            prof_scope ps(this, "swiglu", (double) (K * ncols * 12));
            launch_swiglu(tv(gt), tv(up), tv(mn), kind == 1 ? &e.q8 : nullptr, kind == 2 ? &e.q8k : nullptr, st_);
        }
        if (kind) act_[mn] = e;
        done_[mj] = true;
        wrote_.push_back(mn);
    }

    // The routing of build_moe_ffn (reference qwen_model.c:551-606 semantics):
    //   probs = soft_max(logits); sel = view(argsort(probs, desc), first k); w = get_rows(probs, sel);
    //   w = div(w, sum_rows(w))
    // ==> one kernel per token writing the k expert ids into sel's rows and the renormalized w, with
    // each op's float roundings. probs, the rest of the argsort and the sum are never stored.
    bool op_moe_route(int i) {
        ggml_tensor * sm = g_->nodes[i];
        const ggml_tensor * lg = sm->src[0];
        float scale, max_bias;
        memcpy(&scale, &sm->op_params[0], 4);
        memcpy(&max_bias, &sm->op_params[1], 4);
        if (sm->src[1] || max_bias != 0.0f || lg->type != GGML_TYPE_F32 || lg->nb[0] != sizeof(float) ||
            lg->ne[2] != 1 || lg->ne[3] != 1 || lg->ne[0] > MOE_ROUTE_MAX_EXPERTS || is_output(i) || users_[i].size() != 2) return false;
        const int64_t E = lg->ne[0], T = lg->ne[1];
        int as = -1, rs = -1;
        for (int u : users_[i]) {
            const ggml_tensor * un = g_->nodes[u];
            if (un->op == GGML_OP_ARGSORT && un->src[0] == sm && un->op_params[0] == GGML_SORT_ORDER_DESC) as = u;
            else if (un->op == GGML_OP_RESHAPE && un->src[0] == sm) rs = u;
        }
        if (as < 0 || rs < 0 || is_output(as) || users_[as].size() != 1) return false;
        ggml_tensor * an = g_->nodes[as];
        const int vs = users_[as][0];
        const ggml_tensor * vn = g_->nodes[vs];
        if (vn->op != GGML_OP_VIEW || vn->src[0] != an || vn->data != an->data || vn->nb[1] != an->nb[1] || vn->ne[1] != T) return false;
        const int64_t k = vn->ne[0];
        if (k < 1 || k > MOE_ROUTE_MAX_K || an->nb[0] != sizeof(int32_t)) return false;
        const int gs = sole_user(rs);
        if (gs < 0) return false;
        const ggml_tensor * gn = g_->nodes[gs];
        if (gn->op != GGML_OP_GET_ROWS || gn->src[0] != g_->nodes[rs] || gn->src[1] != vn) return false;
        const int w2 = sole_user(gs);
        if (w2 < 0 || g_->nodes[w2]->op != GGML_OP_RESHAPE || users_[w2].size() != 2 || is_output(w2)) return false;
        int sr = -1, dv = -1;
        for (int u : users_[w2]) {
            const ggml_tensor * un = g_->nodes[u];
            if (un->op == GGML_OP_SUM_ROWS && un->src[0] == g_->nodes[w2]) sr = u;
            else if (un->op == GGML_OP_DIV && un->src[0] == g_->nodes[w2]) dv = u;
        }
        if (sr < 0 || dv < 0 || sole_user(sr) != dv || g_->nodes[dv]->src[1] != g_->nodes[sr]) return false;
        ggml_tensor * dn = g_->nodes[dv];
        if (dn->ne[0] != k || dn->ne[1] != T || !is_2d_contig(dn)) return false;
        moe_route R{};
        R.logits = (const float *) lg->data;
        R.logits_nb1 = (int64_t) (lg->nb[1] / sizeof(float));
        R.n_expert = (int) E;
        R.k = (int) k;
        R.n_tok = (int) T;
        R.scale = scale;
        R.ids = (int32_t *) an->data;
        R.ids_nb1 = (int64_t) (an->nb[1] / sizeof(int32_t));
        R.w = (float *) dn->data;
        R.w_nb1 = (int64_t) (dn->nb[1] / sizeof(float));
        for (int d : { i, as, vs, rs, gs, w2, sr, dv }) done_[d] = true;
        if (T == 1 && route_deferrable(vs, gs, dv)) {
            // held back for the first mul_mat_id reading the ids (op_gemv), which either routes
            // inside its SwiGLU launch or runs launch_moe_route first
            pending_route_[vn] = R;
            return true;
        }
        run_route(R);
        wrote_.push_back(an);
        wrote_.push_back(dn);
        return true;
    }

    void run_route(const moe_route & R) {
        prof_scope ps(this, "moe_route", (double) (R.n_expert * R.n_tok * 4 + R.k * R.n_tok * 8));
        launch_moe_route(R, st_);
    }

    // A one-token routing (ids view vs, weights dv) may wait for the mul_mat_id that reads it first
    // when only mul_mat_ids read the ids (besides the routing's own get_rows gs) and nothing reads
    // the weights before that node.
    bool route_deferrable(int vs, int gs, int dv) const {
        if (!fuse(FUSE_ROUTEG) || c_.cb || is_output(vs) || is_output(dv)) return false;
        int first = INT_MAX;
        for (int u : users_[vs]) {
            if (u == gs) continue;
            const ggml_tensor * un = g_->nodes[u];
            if (un->op != GGML_OP_MUL_MAT_ID || un->src[2] != g_->nodes[vs] || un->src[0] == g_->nodes[vs] ||
                un->src[1] == g_->nodes[vs]) return false;
            first = std::min(first, u);
        }
        return first != INT_MAX && first_reader(dv) > first;
    }

    // mul(experts [n_embd, k, T], w [1, k, T]) -> views of the k slots -> add chain in slot order
    // (-> residual add)  ==>  one kernel with the same float operations in the same order
    // an rms_norm of x (several rows) whose sole user multiplies by an f32 weight row and whose
    // readers are only GEMVs over K-quant weights: op_rms_norm would normalize and quantize it to
    // Q8_K in an act_quant launch of its own. Returns the norm node, the mul node and eps.
    bool norm_q8k_of(const ggml_tensor * x, int & nn, int & nm, float & eps) const {
        const int xi = node_index(x);
        if (!fuse(FUSE_WSUMQ) || !fuse(FUSE_NORM) || !fuse(FUSE_MC) || xi < 0 || x->type != GGML_TYPE_F32 || !ggml_is_contiguous(x) ||
            x->ne[0] > RMS_NORM_MAX_ROW || ggml_nrows(x) < 2) return false;
        for (int j : users_[xi]) {
            const ggml_tensor * n = g_->nodes[j];
            if (done_[j] || n->op != GGML_OP_RMS_NORM || n->src[0] != x || !ggml_is_contiguous(n)) continue;
            const int u = sole_user(j);
            if (u < 0) continue;
            const ggml_tensor * m = g_->nodes[u];
            const ggml_tensor * w = m->src[1];
            if (m->op != GGML_OP_MUL || m->src[0] != n || w->type != GGML_TYPE_F32 || ggml_nrows(w) != 1 || w->ne[0] != x->ne[0] ||
                !ggml_is_contiguous(w) || !ggml_is_contiguous(m) || m->ne[1] != ggml_nrows(x) ||
                ((uintptr_t) x->data | (uintptr_t) w->data) % 16) continue;
            if (!norm_deferrable(u, x->ne[0]) || wanted_act_kind(u) != 2) continue;
            nn = j;
            nm = u;
            memcpy(&eps, n->op_params, 4);
            return true;
        }
        return false;
    }

    bool op_moe_wsum(int i) {
        const ggml_tensor * m = g_->nodes[i];
        const ggml_tensor * e = m->src[0], * w = m->src[1];
        const int64_t n_embd = e->ne[0], k = e->ne[1], T = e->ne[2];
        if (k < 2 || e->ne[3] != 1 || m->type != GGML_TYPE_F32 || e->type != GGML_TYPE_F32 || w->type != GGML_TYPE_F32) return false;
        if (!ggml_is_contiguous(m) || w->ne[0] != 1 || w->ne[1] != k || w->ne[2] != T || w->nb[0] != sizeof(float)) return false;
        if (e->nb[0] != sizeof(float) || is_output(i) || (int64_t) users_[i].size() != k) return false;
        // the slot views, by offset
        std::vector<int> view(k, -1);
        for (int u : users_[i]) {
            const ggml_tensor * v = g_->nodes[u];
            if (v->op != GGML_OP_VIEW || v->src[0] != m || v->ne[0] != n_embd || v->ne[1] != T || v->ne[2] != 1 ||
                v->nb[1] != m->nb[2]) return false;
            const int64_t off = (const char *) v->data - (const char *) m->data;
            if (off % (int64_t) m->nb[1] || off / (int64_t) m->nb[1] >= k || view[off / m->nb[1]] >= 0) return false;
            view[off / m->nb[1]] = u;
        }
        // the chain add(add(add(v0, v1), v2), ...)
        std::vector<int> chain;
        int cur = view[0];
        for (int64_t sl = 1; sl < k; sl++) {
            const int a = sole_user(cur);
            if (a < 0 || sole_user(view[sl]) != a) return false;
            const ggml_tensor * an = g_->nodes[a];
            if (an->op != GGML_OP_ADD || an->src[0] != g_->nodes[cur] || an->src[1] != g_->nodes[view[sl]]) return false;
            chain.push_back(a);
            cur = a;
        }
        ggml_tensor * last = g_->nodes[cur];
        moe_wsum M{};
        M.e = (const float *) e->data;        // e * w is formed inside the kernel, per slot
        M.e_nb1 = (int64_t) (e->nb[1] / sizeof(float));
        M.e_nb2 = (int64_t) (e->nb[2] / sizeof(float));
        M.w = (const float *) w->data;
        M.w_nb1 = (int64_t) (w->nb[1] / sizeof(float));
        M.w_nb2 = (int64_t) (w->nb[2] / sizeof(float));
        M.n_embd = n_embd;
        M.n_tok = T;
        M.k = (int) k;
        // residual add of the sum
        const int r = sole_user(cur);
        if (r >= 0) {
            ggml_tensor * rn = g_->nodes[r];
            const ggml_tensor * res = rn->src[1];
            if (rn->op == GGML_OP_ADD && rn->src[0] == last && res->type == GGML_TYPE_F32 && ggml_are_same_shape(res, last) &&
                res->nb[0] == sizeof(float) && is_2d_contig(rn)) {
                M.res = (const float *) res->data;
                M.res_nb1 = (int64_t) (res->nb[1] / sizeof(float));
                chain.push_back(r);
                last = rn;
            }
        }
        if (!is_2d_contig(last)) return false;
        M.out = (float *) last->data;
        M.out_nb1 = (int64_t) (last->nb[1] / sizeof(float));
        const double wsum_bytes = (double) (n_embd * k * T * 4 + n_embd * T * 4 * (M.res ? 2 : 1));
        int nn = -1, nm = -1;
        float eps = 0.0f;
        if (T >= 2 && norm_q8k_of(last, nn, nm, eps) && wsum_norm_q8k_supported(M, (const float *) g_->nodes[nm]->src[1]->data)) {
            // the next rms_norm * w, normalized and quantized in the same launch (what op_rms_norm
            // would do in an act_quant launch of its own)
            ggml_tensor * mn = g_->nodes[nm];
            act_entry e = alloc_act(2, n_embd, T);
            {
                prof_scope ps(this, "moe_wsum_q8k", wsum_bytes + (double) (n_embd * 4 + n_embd * T + (n_embd / 256 * 4 + n_embd / 16 * 2) * T));
                launch_wsum_norm_q8k(M, (const float *) mn->src[1]->data, eps, e.q8k, st_);
            }
            act_[mn] = e;
            done_[nn] = done_[nm] = true;
        } else {
            prof_scope ps(this, "moe_wsum", wsum_bytes);
            launch_moe_wsum(M, st_);
        }
        for (int v : view) done_[v] = true;
        for (int a : chain) done_[a] = true;
        wrote_.push_back(last);
        return true;
    }

    // the prefill attention kernel: a row of scores fits its LDS, K and V rows 16-byte aligned
    static bool prefill_attn_ok(int64_t n_kv, int64_t hd, const void * k, size_t k_nb_a, size_t k_nb_b,
                                const void * v, size_t v_nb_a, size_t v_nb_b) {
        return n_kv <= attn_prefill_max_kv((int) hd) && ((uintptr_t) k | (uintptr_t) v) % 16 == 0 &&
               k_nb_a % 16 == 0 && k_nb_b % 16 == 0 && v_nb_a % 16 == 0 && v_nb_b % 16 == 0;
    }

    // K^T Q -> soft_max -> cont(permute(V)) -> V KQ -> permute -> cont  ==>  split-KV attention
    bool match_attention(int i, attn_match & M) const {
        const ggml_tensor * kq = g_->nodes[i];
        const ggml_tensor * kp = kq->src[0];
        const ggml_tensor * qp = kq->src[1];
        if (kp->type != GGML_TYPE_F16 || kp->op != GGML_OP_PERMUTE || qp->type != GGML_TYPE_F32) return false;
        const int sm = sole_user(i);
        if (sm < 0) return false;
        const ggml_tensor * smn = g_->nodes[sm];
        if (smn->op != GGML_OP_SOFT_MAX || smn->src[0] != kq) return false;
        float scale, max_bias;
        memcpy(&scale, &smn->op_params[0], 4);
        memcpy(&max_bias, &smn->op_params[1], 4);
        if (max_bias != 0.0f) return false;
        const int kqv = sole_user(sm);
        if (kqv < 0) return false;
        const ggml_tensor * kqvn = g_->nodes[kqv];
        if (kqvn->op != GGML_OP_MUL_MAT || kqvn->src[1] != smn) return false;
        const ggml_tensor * vt = kqvn->src[0];
        const int vti = node_index(vt);
        if (vt->op != GGML_OP_CONT || vti < 0 || sole_user(vti) != kqv) return false;
        const ggml_tensor * vp = vt->src[0];
        if (vp->op != GGML_OP_PERMUTE || vp->type != GGML_TYPE_F16) return false;
        const int pm = sole_user(kqv);
        if (pm < 0) return false;
        const ggml_tensor * pmn = g_->nodes[pm];
        if (pmn->op != GGML_OP_PERMUTE) return false;
        const int ct = sole_user(pm);
        if (ct < 0) return false;
        const ggml_tensor * ctn = g_->nodes[ct];
        if (ctn->op != GGML_OP_CONT || !is_2d_contig(ctn)) return false;

        const int64_t hd = kp->ne[0], n_kv = kp->ne[1], n_head_kv = kp->ne[2];
        const int64_t n_q = qp->ne[1], n_head = qp->ne[2];
        if (kp->ne[3] != 1 || qp->ne[3] != 1 || qp->ne[0] != hd) return false;
        if (vp->ne[0] != n_kv || vp->ne[1] != hd || vp->ne[2] != n_head_kv) return false;
        if (kp->nb[0] != 2 || vp->nb[1] != 2 || qp->nb[0] != 4) return false;
        if (n_q < 1 || n_head % n_head_kv) return false;
        if (hd != 64 && hd != 96 && hd != 128) return false;
        if (n_q > 4 && !prefill_attn_ok(n_kv, hd, kp->data, kp->nb[1], kp->nb[2], vp->data, vp->nb[0], vp->nb[2]) &&
            n_head / n_head_kv > 8) return false;
        if (n_q <= 4 && n_head / n_head_kv > 8) return false;
        if (ctn->ne[0] != hd * n_head || ctn->ne[1] != n_q) return false;
        const ggml_tensor * mask = smn->src[1];
        if (mask && (mask->ne[0] != n_kv || mask->nb[0] != ggml_type_size(mask->type))) return false;
        // 16-byte alignment of the K rows for the staged loads; 4-byte V rows for half2 loads
        if (((uintptr_t) kp->data) % 16 || kp->nb[1] % 16 || kp->nb[2] % 16) return false;
        if (((uintptr_t) vp->data) % 4 || vp->nb[0] % 4 || vp->nb[2] % 4) return false;
        M.kq = i; M.sm = sm; M.vt = vti; M.kqv = kqv; M.pm = pm; M.ct = ct;
        M.kp = kp; M.qp = qp; M.vp = vp; M.mask = mask; M.scale = scale;
        return true;
    }

    // More queries than the fused decode path takes, over more positions than the prefill kernel
    // holds in LDS (a multi-token step deep into the context): the decode kernels, whose workgroups
    // take 4 queries each, over up to ATT_DECODE_MAX_Q queries per launch, each launch with its own
    // rows of Q, mask and output (same arithmetic per query).
    void attn_decode_grouped(const attn_launch & A0) {
        attn_launch A = A0;
        A.scratch_bytes = attn_scratch_bytes(A0.n_kv, std::min(A0.n_q, ATT_DECODE_MAX_Q), A0.n_head, A0.hd);
        A.scratch = (float *) c_.scratch.alloc((size_t) A.scratch_bytes);
        A.rope = 0;
        for (int q0 = 0; q0 < A0.n_q; q0 += ATT_DECODE_MAX_Q) {
            A.n_q = std::min(ATT_DECODE_MAX_Q, A0.n_q - q0);
            A.q = A0.q + (int64_t) q0 * A0.q_nb2;
            A.mask = A0.mask ? (const char *) A0.mask + (int64_t) q0 * A0.mask_nb1 : nullptr;
            A.out = A0.out + (int64_t) q0 * A0.out_nb1;
            const int64_t K = (int64_t) A0.n_head * A0.hd;
            if (A0.out_q.qs) A.out_q = q8_act{ A0.out_q.qs + q0 * K, A0.out_q.d + q0 * (K / 32), A0.out_q.s + q0 * (K / 32) };
            if (A0.out_q8k.qs) A.out_q8k = q8k_act{ A0.out_q8k.qs + q0 * K, A0.out_q8k.d + q0 * (K / 256), A0.out_q8k.bsums + q0 * (K / 16) };
            launch_attn_decode(A, st_);
        }
    }

    // A one-query attention output read only by GEMVs that take it as doubles: the PV launch adds
    // its chunk partials into an accumulator and those GEMVs' prologue rounds and quantizes it, so
    // the output is never materialized and the combination launch does not run.
    bool acc_output_ok(int ct) const {
        const ggml_tensor * ctn = g_->nodes[ct];
        if (!fuse(FUSE_ACCO) || !fuse(FUSE_NORMQ) || c_.cb || is_output(ct) || users_[ct].empty() || ctn->ne[1] != 1 ||
            ggml_nrows(ctn) != 1) return false;
        for (int u : users_[ct]) {
            const ggml_tensor * n = g_->nodes[u];
            if (n->op != GGML_OP_MUL_MAT || n->src[1] != ctn || n->src[0] == ctn || attn_.count(u) || !gemv_capable(n)) return false;
            gemv_launch P{};
            P.type = n->src[0]->type;
            P.K = (int) n->src[0]->ne[0];
            P.ncols = 1;
            if (!gemv_f64_input_supported(P)) return false;
        }
        return true;
    }

    // the attention output's quantized copy for its GEMV readers, written by the combination launch
    // (Q8_0 blocks, or Q8_K super-blocks when the head dims tile them)
    void attn_quant_out(attn_launch & A, int ct, ggml_tensor * ctn, int n_q) {
        const int kind = wanted_act_kind(ct);
        if (kind == 1) {
            act_entry e = alloc_act(1, ctn->ne[0], n_q);
            A.out_q = e.q8;
            act_[ctn] = e;
        } else if (kind == 2 && (A.n_head * A.hd) % 256 == 0 && 256 % A.hd == 0) {
            act_entry e = alloc_act(2, ctn->ne[0], n_q);
            A.out_q8k = e.q8k;
            act_[ctn] = e;
        }
    }

    void run_attention(const attn_match & M) {
        const ggml_tensor * kp = M.kp, * qp = M.qp, * vp = M.vp, * mask = M.mask;
        ggml_tensor * ctn = g_->nodes[M.ct];
        const int hd = (int) kp->ne[0], n_kv = (int) kp->ne[1], n_head_kv = (int) kp->ne[2];
        const int n_q = (int) qp->ne[1], n_head = (int) qp->ne[2];
        attn_launch A{};
        A.q = (const float *) qp->data;
        A.q_nb1 = (int64_t) (qp->nb[2] / 4);
        A.q_nb2 = (int64_t) (qp->nb[1] / 4);
        A.k = (const __half *) kp->data;
        A.k_nb1 = (int64_t) (kp->nb[2] / 2);
        A.k_nb2 = (int64_t) (kp->nb[1] / 2);
        A.v = (const __half *) vp->data;
        A.v_nb1 = (int64_t) (vp->nb[2] / 2);
        A.v_nb2 = (int64_t) (vp->nb[0] / 2);
        A.mask = mask ? mask->data : nullptr;
        A.mask_f16 = mask && mask->type == GGML_TYPE_F16;
        A.mask_nb1 = mask ? (int64_t) mask->nb[1] : 0;
        A.out = (float *) ctn->data;
        A.out_nb1 = (int64_t) (ctn->nb[1] / 4);
        A.n_kv = n_kv; A.n_q = n_q; A.n_head = n_head; A.n_head_kv = n_head_kv; A.hd = hd;
        A.scale = M.scale;
        if (prope_.anchor == M.kq) {
            A.rope = 1;
            A.rq = prope_.q;
            A.rk = prope_.k;
            A.rv = prope_.v;
            A.qn = prope_.qn;
            A.kn = prope_.kn;
            prope_.anchor = -1;
            // one (cos, sin) table per graph for the rotations of the same positions and parameters
            const size_t nbytes = (size_t) n_q * (A.rq.p.n_dims / 2) * sizeof(float2);
            if (cs_tab_ && cs_pos_ == A.rq.pos && cs_ff_ == A.rq.ff && cs_n_ == n_q &&
                memcmp(&cs_p_, &A.rq.p, sizeof(rope_params)) == 0) {
                A.cs_tab = cs_tab_;
                A.cs_mode = 2;
            } else {
                cs_tab_ = (float2 *) c_.scratch.alloc(nbytes);
                cs_pos_ = A.rq.pos;
                cs_ff_ = A.rq.ff;
                cs_n_ = n_q;
                cs_p_ = A.rq.p;
                A.cs_tab = cs_tab_;
                A.cs_mode = 1;
            }
        }
        const double bytes = (double) n_kv * n_head_kv * hd * 2 * 2 + (double) n_head * hd * n_q * 8 +
                             (mask ? (double) n_kv * n_q * ggml_type_size(mask->type) : 0.0);
        if (n_q > 4 && prefill_attn_ok(n_kv, hd, kp->data, kp->nb[1], kp->nb[2], vp->data, vp->nb[0], vp->nb[2])) {
            prof_scope ps(this, "attn_prefill", bytes);
            launch_attn_prefill(A, st_);
        } else if (n_q > 4) {
            attn_quant_out(A, M.ct, ctn, n_q);
            prof_scope ps(this, "attn_decode", bytes * ((n_q + 3) / 4));
            attn_decode_grouped(A);
        } else {
            A.scratch_bytes = attn_scratch_bytes(n_kv, n_q, n_head, hd);
            A.scratch = (float *) c_.scratch.alloc((size_t) A.scratch_bytes);
            if (n_q == 1 && acc_output_ok(M.ct)) {
                A.acc = (double *) c_.scratch.alloc((size_t) n_head * hd * sizeof(double));
                norm_[ctn] = gemv_norm{ (const float *) A.acc, (int64_t) n_head * hd, nullptr, 0.0f, 0, 1 };
            } else {
                attn_quant_out(A, M.ct, ctn, n_q);
            }
            prof_scope ps(this, A.acc ? "attn_decode_acc" : "attn_decode", bytes);
            launch_attn_decode(A, st_);
        }
        done_[M.kq] = done_[M.sm] = done_[M.vt] = done_[M.kqv] = done_[M.pm] = done_[M.ct] = true;
        wrote_.push_back(ctn);
    }

    void op_flash_attn(ggml_tensor * n) {
        const ggml_tensor * q = n->src[0], * k = n->src[1], * v = n->src[2], * mask = n->src[3];
        float scale, max_bias, softcap;
        memcpy(&scale, &n->op_params[0], 4);
        memcpy(&max_bias, &n->op_params[1], 4);
        memcpy(&softcap, &n->op_params[2], 4);
        const int hd = (int) q->ne[0], n_q = (int) q->ne[1], n_head = (int) q->ne[2];
        const int n_kv = (int) k->ne[1], n_head_kv = (int) k->ne[2];
        const bool ok = max_bias == 0.0f && softcap == 0.0f && k->type == GGML_TYPE_F16 && v->type == GGML_TYPE_F16 &&
                        q->type == GGML_TYPE_F32 && q->nb[0] == 4 && k->nb[0] == 2 && v->nb[0] == 2 && v->ne[0] == hd &&
                        n_q >= 1 && n_head % n_head_kv == 0 &&
                        (n_head / n_head_kv <= 8 ||
                         (n_q > 4 && prefill_attn_ok(n_kv, hd, k->data, k->nb[1], k->nb[2], v->data, v->nb[1], v->nb[2]))) &&
                        (hd == 64 || hd == 96 || hd == 128) && ggml_is_contiguous(n) &&
                        ((uintptr_t) k->data) % 16 == 0 && k->nb[1] % 16 == 0 && k->nb[2] % 16 == 0 &&
                        ((uintptr_t) v->data) % 4 == 0 && v->nb[1] % 4 == 0 && v->nb[2] % 4 == 0 &&
                        (!mask || (mask->ne[0] == n_kv && mask->nb[0] == ggml_type_size(mask->type)));
        if (!ok) HIP_ABORT("flash_attn_ext '%s': unsupported configuration", n->name);
        attn_launch A{};
        A.q = (const float *) q->data;
        A.q_nb1 = (int64_t) (q->nb[2] / 4);
        A.q_nb2 = (int64_t) (q->nb[1] / 4);
        A.k = (const __half *) k->data;
        A.k_nb1 = (int64_t) (k->nb[2] / 2);
        A.k_nb2 = (int64_t) (k->nb[1] / 2);
        A.v = (const __half *) v->data;
        A.v_nb1 = (int64_t) (v->nb[2] / 2);
        A.v_nb2 = (int64_t) (v->nb[1] / 2);
        A.mask = mask ? mask->data : nullptr;
        A.mask_f16 = mask && mask->type == GGML_TYPE_F16;
        A.mask_nb1 = mask ? (int64_t) mask->nb[1] : 0;
        A.out = (float *) n->data;
        A.out_nb1 = (int64_t) (n->nb[2] / 4);
        A.n_kv = n_kv; A.n_q = n_q; A.n_head = n_head; A.n_head_kv = n_head_kv; A.hd = hd;
        A.scale = scale;
        A.skip_masked = 1;
        A.p_f32 = 1;
        const double bytes = (double) n_kv * n_head_kv * hd * 2 * 2 + (double) n_head * hd * n_q * 8;
        if (n_q > 4 && prefill_attn_ok(n_kv, hd, k->data, k->nb[1], k->nb[2], v->data, v->nb[1], v->nb[2])) {
            prof_scope ps(this, "attn_prefill", bytes);
            launch_attn_prefill(A, st_);
            return;
        }
        if (n_q > 4) {
            prof_scope ps(this, "attn_decode", bytes * ((n_q + 3) / 4));
            attn_decode_grouped(A);
            return;
        }
        A.scratch_bytes = attn_scratch_bytes(n_kv, n_q, n_head, hd);
        A.scratch = (float *) c_.scratch.alloc((size_t) A.scratch_bytes);
        prof_scope ps(this, "attn_decode", bytes);
        launch_attn_decode(A, st_);
    }
};

// ---------------------------------------------------------------------------------------------
// backend interface

const char * be_name(ggml_backend_t b) { return ((hip_device *) &dev(((hip_backend_ctx *) b->context)->device))->name; }

void be_free(ggml_backend_t b) {
    hip_backend_ctx * c = (hip_backend_ctx *) b->context;
    dev(c->device);
    HIP_CHECK(hipStreamSynchronize(dev(c->device).stream));
    drained(dev(c->device));
    c->scratch.release();
    for (hipEvent_t e : c->event_pool) HIP_CHECK(hipEventDestroy(e));
    delete c;
    delete b;
}

ggml_backend_buffer_type_t be_buft(ggml_backend_t b) { return ggml_backend_hip_buffer_type(((hip_backend_ctx *) b->context)->device); }

void collect_profile(hip_backend_ctx * c) {
    for (pending_event & p : c->pending) {
        float ms = 0.0f;
        HIP_CHECK(hipEventElapsedTime(&ms, p.a, p.b));
        prof_entry & e = c->prof[p.name];
        e.launches++;
        e.ms += ms;
        e.bytes += p.bytes;
    }
    c->pending.clear();
    c->event_next = 0;
}

// queues the graph's kernels on the device stream; a timed (profiled) compute also waits for them
enum ggml_status be_compute_async(ggml_backend_t b, ggml_cgraph * g) {
    hip_backend_ctx * c = (hip_backend_ctx *) b->context;
    hip_device & d = dev(c->device);
    c->timing = c->profiling && (c->computes++ % c->profile_every) == 0;
    const auto t0 = std::chrono::steady_clock::now();
    g_launch_timing.api_on = c->profiling && !c->timing;
    g_launch_timing.api_ms = 0.0;
    executor ex(*c, g);
    ex.run();
    g_launch_timing.api_on = false;
    if (c->profiling && !c->timing) {
        // host time spent walking the graph and enqueuing its kernels (the "host_enqueue" entry),
        // and the part of it inside the kernel launch calls ("host_launch_calls"), over the
        // profiled computes without events (a timed compute also waits for the device: its events,
        // and a mul_mat_id's distinct-expert count read back to the host)
        prof_entry & e = c->prof["host_enqueue"];
        e.launches++;
        e.ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        prof_entry & l = c->prof["host_launch_calls"];
        l.launches++;
        l.ms += g_launch_timing.api_ms;
    }
    if (c->timing) {
        HIP_CHECK(hipStreamSynchronize(d.stream));
        drained(d);
        collect_profile(c);
    }
    return GGML_STATUS_SUCCESS;
}

enum ggml_status be_compute(ggml_backend_t b, ggml_cgraph * g) {
    const enum ggml_status st = be_compute_async(b, g);
    hip_device & d = dev(((hip_backend_ctx *) b->context)->device);
    HIP_CHECK(hipStreamSynchronize(d.stream));
    drained(d);
    return st;
}

// graph_compute with every kernel's scratch in this device's static array (no allocation)
enum ggml_status compute_static(hip_backend_ctx * c, ggml_cgraph * g) {
    hip_device & d = dev(c->device);
    if (!d.static_scratch) {
        fprintf(stderr, "ggml-hip: graph_compute_static: the static scratch of device %d is not resolved\n", c->device);
        return GGML_STATUS_FAILED;
    }
    if (c->profiling) {
        fprintf(stderr, "ggml-hip: graph_compute_static: profiling creates events; turn it off first\n");
        return GGML_STATUS_FAILED;
    }
    scratch_arena own = std::move(c->scratch);
    c->scratch = scratch_arena{};
    c->scratch.fixed = true;
    c->scratch.chunks.push_back({ d.static_scratch, (size_t) GGML_HIP_STATIC_SCRATCH_BYTES });
    enum ggml_status st = GGML_STATUS_SUCCESS;
    try {
        executor ex(*c, g);
        ex.run();
    } catch (const scratch_overflow & o) {
        fprintf(stderr, "ggml-hip: graph_compute_static: the graph needs more than %d bytes of scratch (at least %zu)\n",
                GGML_HIP_STATIC_SCRATCH_BYTES, o.needed);
        st = GGML_STATUS_ALLOC_FAILED;
    }
    HIP_CHECK(hipStreamSynchronize(d.stream));
    drained(d);
    c->scratch = std::move(own);
    return st;
}

void be_set_eval_callback(ggml_backend_t b, ggml_backend_eval_callback cb, void * user) {
    hip_backend_ctx * c = (hip_backend_ctx *) b->context;
    c->cb = cb;
    c->cb_user = user;
}

void be_sync(ggml_backend_t b) {
    hip_device & d = dev(((hip_backend_ctx *) b->context)->device);
    HIP_CHECK(hipStreamSynchronize(d.stream));
    drained(d);
}

ggml_backend_t hip_init_by_name(const char * params) { return ggml_backend_hip_init(params ? atoi(params) : 0); }

struct hip_register {
    hip_register() { ggml_backend_register("HIP", hip_init_by_name); }
} g_hip_register;

} // namespace

extern "C" {

int ggml_backend_hip_get_device_count(void) { return device_count(); }

void ggml_backend_hip_get_device_description(int device, char * description, size_t description_size) {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, device) != hipSuccess) {
        (void) hipGetLastError();
        snprintf(description, description_size, "unavailable");
        return;
    }
    snprintf(description, description_size, "%s (%s, %d CUs, %.0f GiB)", p.name, p.gcnArchName, p.multiProcessorCount,
             p.totalGlobalMem / 1073741824.0);
}

ggml_backend_buffer_type_t ggml_backend_hip_buffer_type(int device) {
    hip_device & d = devices()[device];
    if (!d.buft.context) {
        d.id = device;
        snprintf(d.name, sizeof(d.name), "HIP%d", device);
        d.buft.iface = { buft_name, buft_alloc, buft_align, nullptr, buft_is_host, buft_no_reuse };
        d.buft.context = &d;
    }
    return &d.buft;
}

ggml_backend_t ggml_backend_hip_init(int device) {
    if (device < 0 || device >= device_count()) return nullptr;
    hip_device & d = dev(device);   // makes the device current
    if (!d.static_scratch) {
        void * p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            fprintf(stderr, "ggml-hip: device %d: no address for the static scratch (%s)\n", device, hipGetErrorString(e));
            return nullptr;
        }
        d.static_scratch = (uint8_t *) p;
    }
    ggml_backend_hip_buffer_type(device);
    hip_backend_ctx * c = new hip_backend_ctx();
    c->device = device;
    if (getenv("GGML_HIP_NO_FUSION")) c->fusion = false;
    if (const char * m = getenv("GGML_HIP_FUSE")) c->fuse_mask = atoi(m);
    ggml_backend * b = new ggml_backend();
    b->iface.get_name = be_name;
    b->iface.free = be_free;
    b->iface.get_default_buffer_type = be_buft;
    b->iface.graph_compute = be_compute;
    b->iface.graph_compute_async = be_compute_async;
    b->iface.synchronize = be_sync;
    b->iface.set_eval_callback = be_set_eval_callback;
    b->context = c;
    return b;
}

bool ggml_backend_is_hip(ggml_backend_t backend) { return backend && backend->iface.graph_compute == be_compute; }

enum ggml_status ggml_backend_hip_graph_compute_static(ggml_backend_t backend, struct ggml_cgraph * cgraph) {
    if (!ggml_backend_is_hip(backend) || !cgraph) return GGML_STATUS_FAILED;
    return compute_static((hip_backend_ctx *) backend->context, cgraph);
}

// model.cpp:1675-1728 (see the declaration for the contract)
enum ggml_status ggml_backend_hip_sample(ggml_backend_t backend, const struct ggml_tensor * logits, int64_t row,
                                         const struct ggml_hip_sampler_params * p, const int32_t * recent,
                                         size_t n_recent, double u, int32_t * token, bool * used_draw) {
    auto fail = [](const char * why) {
        fprintf(stderr, "ggml_backend_hip_sample: %s\n", why);
        return GGML_STATUS_FAILED;
    };
    if (!ggml_backend_is_hip(backend)) return fail("not a HIP backend");
    if (!logits || !p || !token || (n_recent && !recent)) return fail("null argument");
    hip_backend_ctx * c = (hip_backend_ctx *) backend->context;
    if (logits->type != GGML_TYPE_F32 || !logits->data || logits->nb[0] != sizeof(float)) return fail("logits must be F32 with contiguous rows");
    if (!logits->buffer || ggml_backend_buffer_get_type(logits->buffer) != ggml_backend_hip_buffer_type(c->device)) {
        return fail("logits are not in this backend's device buffer");
    }
    const int64_t n = logits->ne[0];
    if (n < 1 || n > INT_MAX / 4) return fail("row length out of range");
    if (row < 0 || row >= ggml_nrows(logits)) return fail("row out of range");
    const int64_t i1 = row % logits->ne[1], i2 = (row / logits->ne[1]) % logits->ne[2], i3 = row / (logits->ne[1] * logits->ne[2]);
    const float * base = (const float *) ((const char *) logits->data + i1 * logits->nb[1] + i2 * logits->nb[2] + i3 * logits->nb[3]);

    // the window (model.cpp:1677-1681) as distinct ids with their occurrence counts
    std::vector<int32_t> win;
    if (p->repeat_penalty != 1.0f && n_recent > 0) {
        const size_t start = n_recent > (size_t) p->repeat_last_n ? n_recent - (size_t) p->repeat_last_n : 0;
        for (size_t i = start; i < n_recent; i++) {
            if (recent[i] >= 0 && (int64_t) recent[i] < n) win.push_back(recent[i]);
        }
        std::sort(win.begin(), win.end());
    }
    std::vector<int32_t> table;           // ids, then counts
    int n_pen = 0;
    for (size_t i = 0; i < win.size();) {
        size_t j = i;
        while (j < win.size() && win[j] == win[i]) j++;
        table.push_back(win[i]);
        n_pen++;
        i = j;
    }
    for (size_t i = 0; i < win.size();) {
        size_t j = i;
        while (j < win.size() && win[j] == win[i]) j++;
        table.push_back((int32_t) (j - i));
        i = j;
    }

    hip_device & d = dev(c->device);
    const size_t ints = 4 + table.size();
    if (ints > d.smp_ints) {
        HIP_CHECK(hipStreamSynchronize(d.stream));
        if (d.smp) HIP_CHECK(hipFree(d.smp));
        d.smp_ints = std::max(ints, (size_t) 4096);
        HIP_CHECK(hipMalloc(&d.smp, d.smp_ints * sizeof(int)));
    }
    if (!table.empty()) {
        const size_t bytes = table.size() * sizeof(int32_t);
        if (uint8_t * slot = upload_slot(d, bytes)) {
            memcpy(slot, table.data(), bytes);
            HIP_CHECK(hipMemcpyAsync(d.smp + 4, slot, bytes, hipMemcpyHostToDevice, d.stream));
        } else {
            HIP_CHECK(hipMemcpyAsync(d.smp + 4, table.data(), bytes, hipMemcpyHostToDevice, d.stream));
            HIP_CHECK(hipStreamSynchronize(d.stream));
        }
    }
    sample_request r;
    r.logits = base;
    r.n = (int) n;
    r.pen_ids = d.smp + 4;
    r.pen_cnt = d.smp + 4 + n_pen;
    r.n_pen = n_pen;
    r.temp = p->temp;
    r.top_k = p->top_k;
    r.top_p = p->top_p;
    r.penalty = p->repeat_penalty;
    r.u = u;
    r.out = d.smp;
    int res[3] = { 0, 0, SMP_OVERFLOW };
    auto read_result = [&]() {
        int * area = (int *) download_area(d, sizeof(res));
        HIP_CHECK(hipMemcpyAsync(area, d.smp, sizeof(res), hipMemcpyDeviceToHost, d.stream));
        HIP_CHECK(hipStreamSynchronize(d.stream));
        drained(d);
        memcpy(res, area, sizeof(res));
    };
    if (sample_fast_path(r)) {
        launch_sample(r, d.stream);
        read_result();
    }
    if (res[2] == SMP_OVERFLOW) {
        const size_t ws = sample_sorted_ws_bytes((int) n);
        if (ws > d.smp_ws_size) {
            HIP_CHECK(hipStreamSynchronize(d.stream));
            if (d.smp_ws) HIP_CHECK(hipFree(d.smp_ws));
            d.smp_ws_size = ws;
            HIP_CHECK(hipMalloc(&d.smp_ws, ws));
        }
        launch_sample_sorted(r, d.smp_ws, d.smp_ws_size, d.stream);
        read_result();
    }
    if (res[2] == SMP_NONFINITE) return fail("the largest logit is not finite");
    if (res[2] != SMP_OK) return fail("sampling kernel reported an error");
    *token = res[0];
    if (used_draw) *used_draw = res[1] != 0;
    return GGML_STATUS_SUCCESS;
}

void ggml_backend_hip_set_fusion(ggml_backend_t backend, bool enable) {
    if (ggml_backend_is_hip(backend)) ((hip_backend_ctx *) backend->context)->fusion = enable;
}
void ggml_backend_hip_set_profiling(ggml_backend_t backend, bool enable) {
    if (ggml_backend_is_hip(backend)) ((hip_backend_ctx *) backend->context)->profiling = enable;
}
void ggml_backend_hip_set_profile_sampling(ggml_backend_t backend, int every) {
    if (ggml_backend_is_hip(backend)) ((hip_backend_ctx *) backend->context)->profile_every = every > 1 ? every : 1;
}
void ggml_backend_hip_set_profile_filter(ggml_backend_t backend, const char * prefix) {
    if (ggml_backend_is_hip(backend)) ((hip_backend_ctx *) backend->context)->profile_filter = prefix ? prefix : "";
}
void ggml_backend_hip_reset_profile(ggml_backend_t backend) {
    if (ggml_backend_is_hip(backend)) ((hip_backend_ctx *) backend->context)->prof.clear();
}
int ggml_backend_hip_profile_count(ggml_backend_t backend) {
    return ggml_backend_is_hip(backend) ? (int) ((hip_backend_ctx *) backend->context)->prof.size() : 0;
}
bool ggml_backend_hip_profile_entry(ggml_backend_t backend, int i, char * name, size_t name_size,
                                    int64_t * launches, double * total_ms, double * total_bytes) {
    if (!ggml_backend_is_hip(backend)) return false;
    hip_backend_ctx * c = (hip_backend_ctx *) backend->context;
    if (i < 0 || i >= (int) c->prof.size()) return false;
    auto it = c->prof.begin();
    std::advance(it, i);
    snprintf(name, name_size, "%s", it->first.c_str());
    *launches = it->second.launches;
    *total_ms = it->second.ms;
    *total_bytes = it->second.bytes;
    return true;
}

} // extern "C"
