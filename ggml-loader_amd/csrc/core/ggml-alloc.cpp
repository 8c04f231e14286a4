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
#include <unordered_map>
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
};

static void plan_graph(ggml_gallocr * ga, ggml_cgraph * g) {
    ga->offsets.clear();
    std::unordered_map<ggml_tensor *, int> last_use;
    for (int i = 0; i < g->n_nodes; i++) {
        ggml_tensor * n = g->nodes[i];
        for (int s = 0; s < GGML_MAX_SRC; s++) {
            if (n->src[s]) last_use[base_of(n->src[s])] = i;
        }
        if (n->view_src) last_use[n->view_src] = std::max(last_use[n->view_src], i);
    }
    arena a(ga->alignment);
    std::unordered_map<ggml_tensor *, size_t> placed;
    auto place = [&](ggml_tensor * t) {
        if (!needs_alloc(t) || placed.count(t)) return;
        const size_t sz = ggml_backend_buft_get_alloc_size(ga->buft, t);
        const size_t off = a.alloc(sz);
        placed[t] = off;
        ga->offsets.push_back({ t, off });
    };
    for (int i = 0; i < g->n_leafs; i++) place(g->leafs[i]);
    // frees scheduled per node index
    std::vector<std::vector<ggml_tensor *>> frees(g->n_nodes);
    for (int i = 0; i < g->n_nodes; i++) {
        ggml_tensor * n = g->nodes[i];
        if (!needs_alloc(n)) continue;
        if (n->flags & GGML_TENSOR_FLAG_OUTPUT) continue;
        if (i == g->n_nodes - 1) continue;
        auto it = last_use.find(n);
        if (it == last_use.end()) continue; // unconsumed: graph output
        frees[it->second].push_back(n);
    }
    const bool reuse = !(ga->buft->iface.no_reuse && ga->buft->iface.no_reuse(ga->buft));
    for (int i = 0; i < g->n_nodes; i++) {
        place(g->nodes[i]);
        if (!reuse) continue;
        for (ggml_tensor * t : frees[i]) {
            if (t == g->nodes[i]) continue;
            a.release(placed[t], ggml_backend_buft_get_alloc_size(ga->buft, t));
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
