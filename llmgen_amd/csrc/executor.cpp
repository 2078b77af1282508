// executor.cpp -- the host-side executor slice around the attention path (C++ restatement of the parts of
// src/executor.zig that feed the attention kernels): packed step metadata, StepState binding, the per-layer
// attention dispatch, pass splitting and decode graph buckets.  The C-ABI is declared in include/llmgen_host.h.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "llmgen_attn.h"
#include "llmgen_host.h"
#include "llmgen_model.h"

namespace {

constexpr uint64_t SEED_STEP = 0x9E3779B97F4A7C15ull;  // executor.zig:773

int32_t *i32_at(uint8_t *base, size_t off) { return reinterpret_cast<int32_t *>(base + off); }
float *f32_at(uint8_t *base, size_t off) { return reinterpret_cast<float *>(base + off); }

}  // namespace

extern "C" {

llmgen_layout llmgen_layout_init(size_t n_tok, size_t n_seq, size_t n_tiles, size_t max_blocks) {
    llmgen_layout l{};
    size_t off = 8;  // the first 8 bytes hold the step seed (u64)
    l.seed = 0;
    l.ids = off;
    off += 4 * n_tok;
    l.pos = off;
    off += 4 * n_tok;
    l.slots = off;
    off += 4 * n_tok;
    l.cu_q = off;
    off += 4 * (n_seq + 1);
    l.ctx = off;
    off += 4 * n_seq;
    l.last = off;
    off += 4 * n_seq;
    l.temps = off;
    off += 4 * n_seq;
    l.tile_seq = off;
    off += 4 * n_tiles;
    l.tile_q0 = off;
    off += 4 * n_tiles;
    l.bt = off;
    off += 4 * n_seq * max_blocks;
    l.total = off;
    return l;
}

int llmgen_entry_emits(const llmgen_seq *seqs, const llmgen_entry *e) {
    return e->q_start + e->q_len == seqs[e->seq].n_tokens;
}

int llmgen_step_is_decode(const llmgen_seq *seqs, const llmgen_entry *entries, int n_entries) {
    for (int i = 0; i < n_entries; ++i)
        if (!(entries[i].q_len == 1 && llmgen_entry_emits(seqs, &entries[i]))) return 0;
    return 1;
}

int llmgen_step_tiles(const llmgen_entry *entries, int n_entries, int pf_tile) {
    if (pf_tile <= 0) return -1;
    int n = 0;
    for (int i = 0; i < n_entries; ++i) n += (entries[i].q_len + pf_tile - 1) / pf_tile;
    return n;
}

int llmgen_single_rows(const llmgen_entry *entries, int n_entries, int seq_num) {
    int n = seq_num > n_entries ? seq_num - n_entries : 0;
    for (int i = 0; i < n_entries; ++i) n += entries[i].q_len == 1;
    return n;
}

int llmgen_fill_meta(uint8_t *meta_host, llmgen_layout lay, const llmgen_seq *seqs, const llmgen_entry *entries,
                     int n_entries, int seq_num, int n_tiles, int pf_tile, int block_size, int max_blocks,
                     uint64_t *step_seed) {
    if (!meta_host || seq_num < n_entries || block_size <= 0 || max_blocks < 0 || pf_tile <= 0 || !step_seed)
        return -1;
    *step_seed += SEED_STEP;
    memcpy(meta_host + lay.seed, step_seed, 8);
    int32_t *ids = i32_at(meta_host, lay.ids), *pos = i32_at(meta_host, lay.pos);
    int32_t *slots = i32_at(meta_host, lay.slots), *cu_q = i32_at(meta_host, lay.cu_q);
    int32_t *ctx = i32_at(meta_host, lay.ctx), *last = i32_at(meta_host, lay.last);
    float *temps = f32_at(meta_host, lay.temps);
    int32_t *tseq = i32_at(meta_host, lay.tile_seq), *tq0 = i32_at(meta_host, lay.tile_q0);
    int32_t *bt = i32_at(meta_host, lay.bt);
    const size_t n_tok_cap = (lay.pos - lay.ids) / 4, n_seq_cap = (lay.ctx - lay.cu_q) / 4 - 1;
    if ((size_t)seq_num > n_seq_cap) return -2;
    size_t t = 0;
    int tile = 0;
    cu_q[0] = 0;
    for (int si = 0; si < n_entries; ++si) {
        const llmgen_entry &e = entries[si];
        const llmgen_seq &sq = seqs[e.seq];
        if (e.q_start < 0 || e.q_len < 0 || e.q_start + e.q_len > sq.n_tokens || sq.n_blocks > max_blocks) return -3;
        if (t + e.q_len > n_tok_cap) return -4;
        for (int j = 0; j < e.q_len; ++j) {
            const int p = e.q_start + j;
            if (p / block_size >= sq.n_blocks) return -5;
            ids[t] = sq.token_ids[p];
            pos[t] = p;
            slots[t] = sq.block_table[p / block_size] * block_size + p % block_size;  // batching.zig:74-77
            ++t;
        }
        cu_q[si + 1] = (int32_t)t;
        ctx[si] = e.q_start + e.q_len;
        last[si] = (int32_t)t - 1;
        temps[si] = sq.temperature;
        int32_t *row = bt + (size_t)si * max_blocks;
        memcpy(row, sq.block_table, sizeof(int32_t) * sq.n_blocks);
        memset(row + sq.n_blocks, 0, sizeof(int32_t) * (max_blocks - sq.n_blocks));
        if (n_tiles > 0) {
            for (int q0 = 0; q0 < e.q_len; q0 += pf_tile) {
                if (tile >= n_tiles) return -6;
                tseq[tile] = si;
                tq0[tile] = q0;
                ++tile;
            }
        }
    }
    // graph-bucket padding rows: ctx 0 (attention writes zeros), slot -1 (no KV write).  In a step with prefill
    // tiles each padding row also gets a tile, so that the kernels write its zero row.
    for (int s = n_entries; s < seq_num; ++s) {
        if (t >= n_tok_cap) return -4;
        ids[t] = 0;
        pos[t] = 0;
        slots[t] = -1;
        ++t;
        cu_q[s + 1] = (int32_t)t;
        ctx[s] = 0;
        last[s] = (int32_t)t - 1;
        temps[s] = 0.f;
        memset(bt + (size_t)s * max_blocks, 0, sizeof(int32_t) * max_blocks);
        if (n_tiles > 0) {
            if (tile >= n_tiles) return -6;
            tseq[tile] = s;
            tq0[tile] = 0;
            ++tile;
        }
    }
    // Single-row tiles (decode and padding rows) first, then the multi-row tiles; each part lightest first, by the
    // keys a tile needs (stable: entry order among equals).  The reference lists tiles in entry order.  The kernels
    // accept any order: they walk each part from its end, so the longest decode rows and the heaviest prefill
    // tiles (a long prompt's last ones) start first, and the single-row count hip_attn_prefill_rows takes marks
    // where the parts meet.
    if (tile > 1) {
        std::vector<int> order(tile);
        std::vector<int32_t> kend(tile), s0(tseq, tseq + tile), q00(tq0, tq0 + tile);
        for (int i = 0; i < tile; ++i) {
            const int si = s0[i], q_len = cu_q[si + 1] - cu_q[si];
            kend[i] = ctx[si] - q_len + std::min(q00[i] + pf_tile, q_len);
            order[i] = i;
        }
        std::vector<char> multi(tile);
        for (int i = 0; i < tile; ++i) multi[i] = cu_q[s0[i] + 1] - cu_q[s0[i]] > 1;
        std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
            return multi[a] != multi[b] ? multi[a] < multi[b] : kend[a] < kend[b];
        });
        for (int i = 0; i < tile; ++i) {
            tseq[i] = s0[order[i]];
            tq0[i] = q00[order[i]];
        }
    }
    return llmgen_single_rows(entries, n_entries, seq_num);
}

void llmgen_bind_step(llmgen_step_state *st, void *meta_dev, llmgen_layout lay, int n_tok, int n_seq, int n_tiles,
                      int decode, int hidden, int n_head, int n_kv_head, int head_dim, int block_size, int max_blocks,
                      size_t max_model_len, void *part_o, void *part_ml, void *sample_scratch, int single_rows) {
    uint8_t *m = static_cast<uint8_t *>(meta_dev);
    st->n_tok = n_tok;
    st->n_seq = n_seq;
    st->n_tiles = n_tiles;
    st->decode = decode;
    st->hidden = hidden;
    st->n_head = n_head;
    st->n_kv_head = n_kv_head;
    st->head_dim = head_dim;
    st->attn_scale = 1.0f / sqrtf((float)head_dim);
    st->block_size = block_size;
    st->max_blocks = max_blocks;
    st->max_model_len = max_model_len;
    st->seed = m + lay.seed;
    st->pos = m + lay.pos;
    st->slots = m + lay.slots;
    st->cu_q = m + lay.cu_q;
    st->ctx = m + lay.ctx;
    st->last = m + lay.last;
    st->temps = m + lay.temps;
    st->tile_seq = m + lay.tile_seq;
    st->tile_q0 = m + lay.tile_q0;
    st->block_tables = m + lay.bt;
    st->cos_sin = nullptr;
    st->part_o = part_o;
    st->part_ml = part_ml;
    st->sample_scratch = sample_scratch;
    st->single_rows = single_rows;
}

int llmgen_part_size(int n_seq) {
    if (n_seq >= 64) return 512;
    if (n_seq >= 16) return 256;
    if (n_seq >= 4) return 128;
    return 64;
}

int llmgen_max_parts(int n_seq, size_t max_model_len) {
    const int ps = llmgen_part_size(n_seq);
    return (int)((max_model_len + ps - 1) / ps);
}

int llmgen_paged_attention(const llmgen_step_state *st, uint16_t *out, const uint16_t *q, const uint16_t *k,
                           const uint16_t *v, uint16_t *k_cache, uint16_t *v_cache, int store_kv) {
    if (!st || !out || !q || !k_cache || !v_cache) return -1;
    const int32_t *slots = static_cast<const int32_t *>(st->slots);
    const int32_t *bt = static_cast<const int32_t *>(st->block_tables);
    const int32_t *ctx = static_cast<const int32_t *>(st->ctx);
    if (st->decode) {
        const int ps = llmgen_part_size(st->n_seq), mp = llmgen_max_parts(st->n_seq, st->max_model_len);
        float *po = static_cast<float *>(st->part_o), *pml = static_cast<float *>(st->part_ml);
        if (store_kv) {
            if (!k || !v) return -1;
            hip_attn_decode_store_kv(out, q, k, v, slots, k_cache, v_cache, bt, ctx, st->n_seq, st->n_head,
                                     st->n_kv_head, st->head_dim, st->max_blocks, st->block_size, st->attn_scale, po,
                                     pml, ps, mp);
        } else {
            hip_attn_decode(out, q, k_cache, v_cache, bt, ctx, st->n_seq, st->n_head, st->n_kv_head, st->head_dim,
                            st->max_blocks, st->block_size, st->attn_scale, po, pml, ps, mp);
        }
        return 0;
    }
    if (store_kv) {
        if (!k || !v) return -1;
        hip_store_kv(k, v, slots, k_cache, v_cache, st->n_tok, st->n_kv_head, st->head_dim, st->block_size);
    }
    hip_attn_prefill_rows(out, q, k_cache, v_cache, bt, ctx, static_cast<const int32_t *>(st->cu_q),
                          static_cast<const int32_t *>(st->tile_seq), static_cast<const int32_t *>(st->tile_q0),
                          st->n_tiles, st->n_head, st->n_kv_head, st->head_dim, st->max_blocks, st->block_size,
                          st->attn_scale, st->single_rows);
    return 0;
}

void llmgen_workspace(int n_head, int head_dim, int max_seqs, size_t max_tokens, size_t max_model_len,
                      int block_size, int pf_tile, size_t out[4]) {
    const size_t max_blocks = (max_model_len + block_size - 1) / block_size;
    out[0] = llmgen_layout_init(max_tokens, max_seqs, max_tokens / pf_tile + max_seqs, max_blocks).total;
    size_t cap = 0;
    for (int s = 1; s <= max_seqs; ++s) cap = std::max(cap, (size_t)s * llmgen_max_parts(s, max_model_len));
    out[1] = cap * n_head * head_dim * 4;
    out[2] = cap * n_head * 2 * 4;
    out[3] = hip_sample_scratch_bytes(max_seqs);
}

int llmgen_decode_buckets(int max_seqs, int *out, int cap) {
    std::vector<int> b;
    for (int x : {1, 2, 4, 8})
        if (x <= max_seqs) b.push_back(x);
    for (int x = 16; x <= max_seqs; x += 16) b.push_back(x);
    if (b.empty() || b.back() != max_seqs) b.push_back(max_seqs);
    if ((int)b.size() > cap) return -1;
    std::copy(b.begin(), b.end(), out);
    return (int)b.size();
}

int llmgen_plan_passes(const llmgen_entry *entries, int n_entries, size_t max_tokens, llmgen_entry *pieces,
                       int *owner, int *pass, int cap) {
    if (max_tokens == 0) return -1;
    int n = 0, p = 0;
    size_t room = max_tokens;
    for (int idx = 0; idx < n_entries; ++idx) {
        int start = entries[idx].q_start, left = entries[idx].q_len;
        while (left > 0) {
            const int take = (int)std::min<size_t>(left, room);
            if (n >= cap) return -1;
            pieces[n] = llmgen_entry{entries[idx].seq, start, take};
            owner[n] = idx;
            pass[n] = p;
            ++n;
            start += take;
            left -= take;
            room -= take;
            if (room == 0) {  // flushPass
                ++p;
                room = max_tokens;
            }
        }
    }
    return n;
}

}  // extern "C"

// ------------------------------------------------------------------------------------------------------------
// Decode graph buckets
// ------------------------------------------------------------------------------------------------------------
namespace {

struct Bucket {
    int size = 0;
    llmgen_layout lay{};
    uint8_t *meta_dev = nullptr;
    uint16_t *q = nullptr, *k = nullptr, *v = nullptr, *out = nullptr;
    float *part_o = nullptr, *part_ml = nullptr;
    hipGraphExec_t exec = nullptr;
};

struct Graphs {
    int n_layers, nq, nkv, hd, block_size, max_blocks;
    size_t max_model_len;
    std::vector<uint16_t *> kc, vc;
    std::vector<Bucket> buckets;
    uint8_t *meta_host = nullptr;  // pinned, sized for the largest bucket
    uint64_t step_seed = 0;
    int last = -1;
};

bool ok(hipError_t e, const char *what) {
    if (e == hipSuccess) return true;
    fprintf(stderr, "[llmgen-host] %s: %s\n", what, hipGetErrorString(e));
    return false;
}

void run_nodes(Graphs &g, Bucket &b, int n_seq) {
    llmgen_step_state st{};
    llmgen_bind_step(&st, b.meta_dev, b.lay, n_seq, n_seq, 0, 1, 0, g.nq, g.nkv, g.hd, g.block_size, g.max_blocks,
                     g.max_model_len, b.part_o, b.part_ml, nullptr, n_seq);
    for (int l = 0; l < g.n_layers; ++l) llmgen_paged_attention(&st, b.out, b.q, b.k, b.v, g.kc[l], g.vc[l], 1);
}

void free_bucket(Bucket &b) {
    if (b.exec) (void)hipGraphExecDestroy(b.exec);
    for (void *p : {(void *)b.meta_dev, (void *)b.q, (void *)b.k, (void *)b.v, (void *)b.out, (void *)b.part_o,
                    (void *)b.part_ml})
        if (p) (void)hipFree(p);
    b = Bucket{};
}

}  // namespace

extern "C" {

void llmgen_graphs_destroy(void *graphs) {
    Graphs *g = static_cast<Graphs *>(graphs);
    if (!g) return;
    (void)hipStreamSynchronize((hipStream_t)hip_get_stream());
    for (Bucket &b : g->buckets) free_bucket(b);
    if (g->meta_host) (void)hipHostFree(g->meta_host);
    delete g;
}

void *llmgen_graphs_create(int n_layers, uint16_t *const *k_caches, uint16_t *const *v_caches, int n_head,
                           int n_kv_head, int head_dim, int block_size, size_t max_model_len, int max_seqs,
                           const int *buckets, int n_buckets) {
    if (n_layers <= 0 || !k_caches || !v_caches || n_head <= 0 || n_kv_head <= 0 || block_size <= 0 ||
        max_seqs <= 0)
        return nullptr;
    hipStream_t stream = (hipStream_t)hip_get_stream();
    if (!stream) {
        fprintf(stderr, "[llmgen-host] graphs need a capturable stream: call hip_init or hip_set_stream first\n");
        return nullptr;
    }
    Graphs *g = new Graphs{};
    g->n_layers = n_layers;
    g->nq = n_head;
    g->nkv = n_kv_head;
    g->hd = head_dim;
    g->block_size = block_size;
    g->max_model_len = max_model_len;
    g->max_blocks = (int)((max_model_len + block_size - 1) / block_size);
    g->kc.assign(k_caches, k_caches + n_layers);
    g->vc.assign(v_caches, v_caches + n_layers);
    std::vector<int> sizes;
    if (buckets && n_buckets > 0) {
        sizes.assign(buckets, buckets + n_buckets);
    } else {
        sizes.resize(64);
        const int n = llmgen_decode_buckets(max_seqs, sizes.data(), 64);
        if (n < 0) {
            delete g;
            return nullptr;
        }
        sizes.resize(n);
    }
    std::sort(sizes.begin(), sizes.end());
    size_t meta_max = 0;
    for (int bs : sizes) meta_max = std::max(meta_max, llmgen_layout_init(bs, bs, 0, g->max_blocks).total);
    if (!ok(hipHostMalloc((void **)&g->meta_host, meta_max, hipHostMallocDefault), "hipHostMalloc")) {
        delete g;
        return nullptr;
    }
    for (int bs : sizes) {
        Bucket b;
        b.size = bs;
        b.lay = llmgen_layout_init(bs, bs, 0, g->max_blocks);
        const size_t qb = (size_t)bs * n_head * head_dim * 2, kb = (size_t)bs * n_kv_head * head_dim * 2;
        const size_t cap = (size_t)bs * llmgen_max_parts(bs, max_model_len);
        bool good = ok(hipMalloc((void **)&b.meta_dev, b.lay.total), "hipMalloc") &&
                    ok(hipMalloc((void **)&b.q, qb), "hipMalloc") && ok(hipMalloc((void **)&b.out, qb), "hipMalloc") &&
                    ok(hipMalloc((void **)&b.k, kb), "hipMalloc") && ok(hipMalloc((void **)&b.v, kb), "hipMalloc") &&
                    ok(hipMalloc((void **)&b.part_o, cap * n_head * head_dim * 4), "hipMalloc") &&
                    ok(hipMalloc((void **)&b.part_ml, cap * n_head * 2 * 4), "hipMalloc");
        if (good) {
            good = ok(hipMemsetAsync(b.q, 0, qb, stream), "memset") && ok(hipMemsetAsync(b.k, 0, kb, stream), "memset") &&
                   ok(hipMemsetAsync(b.v, 0, kb, stream), "memset");
        }
        if (good) {
            // warm-up with padding rows only (ctx 0, slot -1: no KV is read or written), then capture
            uint64_t seed = 0;
            llmgen_fill_meta(g->meta_host, b.lay, nullptr, nullptr, 0, bs, 0, 64, block_size, g->max_blocks, &seed);
            good = ok(hipMemcpyAsync(b.meta_dev, g->meta_host, b.lay.total, hipMemcpyHostToDevice, stream), "h2d") &&
                   ok(hipStreamSynchronize(stream), "sync");
        }
        if (good) {
            run_nodes(*g, b, bs);
            good = ok(hipStreamSynchronize(stream), "warm-up");
        }
        if (good && hip_graph_begin() == 0) {
            run_nodes(*g, b, bs);
            b.exec = (hipGraphExec_t)hip_graph_end();
            good = b.exec != nullptr;
        } else {
            good = false;
        }
        if (!good) {
            free_bucket(b);
            llmgen_graphs_destroy(g);
            return nullptr;
        }
        g->buckets.push_back(b);
    }
    return g;
}

int llmgen_graphs_step(void *graphs, const llmgen_seq *seqs, const llmgen_entry *entries, int n_entries,
                       const uint16_t *q_dev, const uint16_t *k_dev, const uint16_t *v_dev, uint16_t *out_dev) {
    Graphs *g = static_cast<Graphs *>(graphs);
    if (!g || n_entries <= 0 || !llmgen_step_is_decode(seqs, entries, n_entries)) return -1;
    int bi = -1;
    for (size_t i = 0; i < g->buckets.size(); ++i)
        if (g->buckets[i].size >= n_entries) {
            bi = (int)i;
            break;
        }
    if (bi < 0) return -2;
    Bucket &b = g->buckets[bi];
    hipStream_t stream = (hipStream_t)hip_get_stream();
    // the previous step's upload must have left the pinned buffer before it is rewritten
    if (!ok(hipStreamSynchronize(stream), "sync")) return -3;
    if (llmgen_fill_meta(g->meta_host, b.lay, seqs, entries, n_entries, b.size, 0, 64, g->block_size, g->max_blocks,
                         &g->step_seed) < 0)
        return -4;
    const size_t qrow = (size_t)g->nq * g->hd * 2, krow = (size_t)g->nkv * g->hd * 2;
    bool good = ok(hipMemcpyAsync(b.meta_dev, g->meta_host, b.lay.total, hipMemcpyHostToDevice, stream), "h2d") &&
                ok(hipMemcpyAsync(b.q, q_dev, qrow * n_entries, hipMemcpyDeviceToDevice, stream), "d2d") &&
                ok(hipMemcpyAsync(b.k, k_dev, krow * n_entries, hipMemcpyDeviceToDevice, stream), "d2d") &&
                ok(hipMemcpyAsync(b.v, v_dev, krow * n_entries, hipMemcpyDeviceToDevice, stream), "d2d");
    if (!good) return -3;
    hip_graph_launch(b.exec);
    if (out_dev && !ok(hipMemcpyAsync(out_dev, b.out, qrow * n_entries, hipMemcpyDeviceToDevice, stream), "d2d"))
        return -3;
    g->last = bi;
    return b.size;
}

int llmgen_graphs_replay(void *graphs) {
    Graphs *g = static_cast<Graphs *>(graphs);
    if (!g || g->last < 0) return -1;
    hip_graph_launch(g->buckets[g->last].exec);
    return g->buckets[g->last].size;
}

}  // extern "C"
