// ggml-alloc.cpp — graph activation allocator (ggml_gallocr_*).
//
// Plan for one graph: graph inputs (data-less leafs) get private slots for the whole graph; every
// data-less node gets a slot when it is produced and returns it to a best-fit free list after its
// last consumer has run. Views take their storage from their base tensor, so a view's consumers
// extend the base's lifetime. Nodes nobody consumes (graph outputs) and nodes flagged OUTPUT are
// never recycled. The planned peak becomes one backend buffer that is reused across calls and
// only grows (forward_step replans every token, model.cpp:1561-1566).
#include "ggml-alloc.h"
#include "ggml-backend-impl.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstdint>
#include <vector>

namespace {

struct free_block { size_t off, size; };

class arena {
public:
    explicit arena(size_t align) : align_(align) {}
    size_t alloc(size_t size) {
        size = GGML_PAD(size ? size : 1, align_);
        int best = -1;
        for (int i = 0; i < (int) blocks_.size(); i++) {
            if (blocks_[i].size >= size && (best < 0 || blocks_[i].size < blocks_[best].size)) best = i;
        }
        if (best >= 0) {
            const size_t off = blocks_[best].off;
            blocks_[best].off += size;
            blocks_[best].size -= size;
            if (blocks_[best].size == 0) blocks_.erase(blocks_.begin() + best);
            return off;
        }
        // grow at the end; absorb a trailing free block that touches the end
        size_t off = end_;
        if (!blocks_.empty() && blocks_.back().off + blocks_.back().size == end_) {
            off = blocks_.back().off;
            blocks_.pop_back();
        }
        end_ = off + size;
        peak_ = std::max(peak_, end_);
        return off;
    }
    void release(size_t off, size_t size) {
        size = GGML_PAD(size ? size : 1, align_);
        auto it = std::lower_bound(blocks_.begin(), blocks_.end(), off,
                                   [](const free_block & b, size_t o) { return b.off < o; });
        it = blocks_.insert(it, { off, size });
        // merge with the next, then the previous block
        size_t i = (size_t) (it - blocks_.begin());
        if (i + 1 < blocks_.size() && blocks_[i].off + blocks_[i].size == blocks_[i + 1].off) {
            blocks_[i].size += blocks_[i + 1].size;
            blocks_.erase(blocks_.begin() + i + 1);
        }
        if (i > 0 && blocks_[i - 1].off + blocks_[i - 1].size == blocks_[i].off) {
            blocks_[i - 1].size += blocks_[i].size;
            blocks_.erase(blocks_.begin() + i);
        }
    }
    size_t peak() const { return peak_; }
private:
    size_t align_;
    size_t end_ = 0, peak_ = 0;
    std::vector<free_block> blocks_;
};

inline ggml_tensor * base_of(ggml_tensor * t) { return t->view_src ? t->view_src : t; }
inline bool needs_alloc(const ggml_tensor * t) { return t->data == nullptr && t->view_src == nullptr; }

} // namespace

struct ggml_gallocr {
    ggml_backend_buffer_type_t buft;
    ggml_backend_buffer_t buffer = nullptr;
    size_t alignment = 0;
    // plan of the last graph
    std::vector<std::pair<ggml_tensor *, size_t>> offsets;
    size_t plan_size = 0;
    // planning tables, kept across calls (a graph is replanned every decode step): an
    // open-addressing map tensor -> slot, and per slot its last consumer, offset and the next
    // slot freed after the same node
    std::vector<ggml_tensor *> keys;
    std::vector<int> last_use, free_next, free_head;
    std::vector<size_t> off;
    std::vector<char> placed;
};

static int slot_of(ggml_gallocr * ga, ggml_tensor * t) {
    const size_t mask = ga->keys.size() - 1;
    size_t h = (size_t) ((reinterpret_cast<uintptr_t>(t) >> 4) * 0x9E3779B97F4A7C15ull) & mask;
    for (;; h = (h + 1) & mask) {
        if (ga->keys[h] == t) return (int) h;
        if (!ga->keys[h]) {
            ga->keys[h] = t;
            ga->last_use[h] = -1;
            ga->placed[h] = 0;
            return (int) h;
        }
    }
}

static void plan_graph(ggml_gallocr * ga, ggml_cgraph * g) {
    ga->offsets.clear();
    size_t cap = 64;
    while (cap < 4 * (size_t) (g->n_nodes + g->n_leafs)) cap <<= 1;
    ga->keys.assign(cap, nullptr);
    ga->last_use.resize(cap);
    ga->free_next.resize(cap);
    ga->off.resize(cap);
    ga->placed.resize(cap);
    ga->free_head.assign((size_t) g->n_nodes, -1);
    for (int i = 0; i < g->n_nodes; i++) {
        ggml_tensor * n = g->nodes[i];
        for (int s = 0; s < GGML_MAX_SRC; s++) {
            if (n->src[s]) ga->last_use[slot_of(ga, base_of(n->src[s]))] = i;
        }
        if (n->view_src) {
            const int k = slot_of(ga, n->view_src);
            ga->last_use[k] = std::max(ga->last_use[k], i);
        }
    }
    arena a(ga->alignment);
    auto place = [&](ggml_tensor * t) {
        if (!needs_alloc(t)) return;
        const int k = slot_of(ga, t);
        if (ga->placed[k]) return;
        const size_t o = a.alloc(ggml_backend_buft_get_alloc_size(ga->buft, t));
        ga->placed[k] = 1;
        ga->off[k] = o;
        ga->offsets.push_back({ t, o });
    };
    for (int i = 0; i < g->n_leafs; i++) place(g->leafs[i]);
    // frees scheduled per node index: a list per consumer node, built from the last node back so
    // each list runs in ascending producer order
    for (int i = g->n_nodes - 2; i >= 0; i--) {
        ggml_tensor * n = g->nodes[i];
        if (!needs_alloc(n) || (n->flags & GGML_TENSOR_FLAG_OUTPUT)) continue;
        const int k = slot_of(ga, n);
        const int lu = ga->last_use[k];
        if (lu < 0) continue; // unconsumed: graph output
        ga->free_next[k] = ga->free_head[lu];
        ga->free_head[lu] = k;
    }
    const bool reuse = !(ga->buft->iface.no_reuse && ga->buft->iface.no_reuse(ga->buft));
    for (int i = 0; i < g->n_nodes; i++) {
        place(g->nodes[i]);
        if (!reuse) continue;
        for (int k = ga->free_head[i]; k >= 0; k = ga->free_next[k]) {
            ggml_tensor * t = ga->keys[k];
            if (t == g->nodes[i]) continue;
            a.release(ga->off[k], ggml_backend_buft_get_alloc_size(ga->buft, t));
        }
    }
    ga->plan_size = a.peak();
}

extern "C" {

ggml_gallocr_t ggml_gallocr_new(ggml_backend_buffer_type_t buft) {
    ggml_gallocr * ga = new ggml_gallocr();
    ga->buft = buft;
    ga->alignment = ggml_backend_buft_get_alignment(buft);
    return ga;
}

void ggml_gallocr_free(ggml_gallocr_t ga) {
    if (!ga) return;
    ggml_backend_buffer_free(ga->buffer);
    delete ga;
}

static bool ensure_buffer(ggml_gallocr * ga, size_t need) {
    if (need == 0) need = ga->alignment;
    if (ga->buffer && ggml_backend_buffer_get_size(ga->buffer) >= need) return true;
    size_t sz = need;
    if (ga->buffer) {
        // grow with headroom: the plan grows a little every decode step as n_kv increases
        sz = std::max(need, ggml_backend_buffer_get_size(ga->buffer) + ggml_backend_buffer_get_size(ga->buffer) / 4);
        ggml_backend_buffer_free(ga->buffer);
        ga->buffer = nullptr;
    }
    ga->buffer = ggml_backend_buft_alloc_buffer(ga->buft, sz);
    if (!ga->buffer) {
        fprintf(stderr, "ggml_gallocr: failed to allocate %s buffer of %zu bytes\n", ggml_backend_buft_name(ga->buft), sz);
        return false;
    }
    return true;
}

bool ggml_gallocr_reserve(ggml_gallocr_t ga, struct ggml_cgraph * g) {
    plan_graph(ga, g);
    return ensure_buffer(ga, ga->plan_size);
}

bool ggml_gallocr_alloc_graph(ggml_gallocr_t ga, struct ggml_cgraph * g) {
    plan_graph(ga, g);
    if (!ensure_buffer(ga, ga->plan_size)) return false;
    char * base = (char *) ggml_backend_buffer_get_base(ga->buffer);
    for (auto & p : ga->offsets) {
        if (ggml_backend_tensor_alloc(ga->buffer, p.first, base + p.second) != GGML_STATUS_SUCCESS) return false;
    }
    auto init_view = [](ggml_tensor * t) {
        if (t->view_src && t->data == nullptr) ggml_backend_view_init(t);
    };
    for (int i = 0; i < g->n_leafs; i++) init_view(g->leafs[i]);
    for (int i = 0; i < g->n_nodes; i++) init_view(g->nodes[i]);
    return true;
}

size_t ggml_gallocr_get_buffer_size(ggml_gallocr_t ga, int buffer_id) {
    (void) buffer_id;
    return ga->buffer ? ggml_backend_buffer_get_size(ga->buffer) : 0;
}

} // extern "C"
