// Host emulation of the append kernel (vspec-engine_amd/csrc/paged_kv.hip kv_append):
// the kernel's own per-item code (append_row.h: append_items / append_item /
// append_chunk), compiled for the CPU against hip/hip_runtime.h of this directory, runs
// every work item of every launch of a recorded append sequence in a chosen order.
// Built with AddressSanitizer, every load and store index the kernel computes is checked
// against the exact extents of the pools and inputs.  Running the same sequence in
// forward, reverse and shuffled orders and comparing the pools shows that no two work
// items of a launch write the same bytes with different values (a GPU race would need
// that); comparing with the oracle shows the bytes are the reference's.
//
//   append_emu <case dir> <order>     order: 0 forward, 1 reverse, s >= 2 shuffled (seed s)
//
// <case dir>/meta.txt : dtype src_dtype num_blocks block_tokens kv_heads head_dim launches
// <case dir>/pool_{k,v,ks,vs}.bin : initial pool bytes (ks/vs for int4 pools)
// <case dir>/L<i>.txt : mode batch n_new max_blocks n_items rope_dim max_pos
//     mode 0: uniform batch (L<i>_start.bin), 1: packed tokens (L<i>_item.bin, L<i>_pos.bin),
//     2: decode step (L<i>_ctx.bin); rope_dim > 0: L<i>_cos.bin, L<i>_sin.bin
// <case dir>/L<i>_tables.bin, L<i>_k.bin, L<i>_v.bin
// Writes <case dir>/out<order>_{k,v,ks,vs}.bin.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <random>
#include <string>
#include <vector>

#include "append_row.h"

using namespace vkv;

static std::vector<uint8_t> read_file(const std::string& path, bool required = true) {
    std::vector<uint8_t> out;
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) {
        if (required) {
            fprintf(stderr, "missing %s\n", path.c_str());
            exit(2);
        }
        return out;
    }
    fseek(f, 0, SEEK_END);
    const long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    out.resize((size_t)n);
    if (n > 0 && fread(out.data(), 1, (size_t)n, f) != (size_t)n) exit(2);
    fclose(f);
    return out;
}

static void write_file(const std::string& path, const void* p, size_t n) {
    FILE* f = fopen(path.c_str(), "wb");
    if (!f || (n && fwrite(p, 1, n, f) != n)) exit(3);
    fclose(f);
}

// a heap copy of exactly n bytes (AddressSanitizer bounds every access by n)
static uint8_t* exact_copy(const std::vector<uint8_t>& v) {
    uint8_t* p = (uint8_t*)malloc(v.size() ? v.size() : 1);
    if (!p) exit(4);
    if (!v.empty()) memcpy(p, v.data(), v.size());
    return p;
}

template <int DT, int SRC>
static void run_launch(const AppendParams& p, int order) {
    const uint64_t total = append_items<DT>(p);
    std::vector<uint64_t> ids(total);
    for (uint64_t i = 0; i < total; ++i) ids[i] = order == 1 ? total - 1 - i : i;
    if (order >= 2) {
        std::mt19937_64 rng((uint64_t)order);
        std::shuffle(ids.begin(), ids.end(), rng);
    }
    for (uint64_t it : ids) append_item<DT, SRC>(p, it);
}

template <int DT>
static void dispatch_src(int src, const AppendParams& p, int order) {
    if (src == VSPEC_KV_F32) run_launch<DT, VSPEC_KV_F32>(p, order);
    else run_launch<DT, VSPEC_KV_F16>(p, order);
}

int main(int argc, char** argv) {
    if (argc != 3) {
        fprintf(stderr, "usage: append_emu <case dir> <order>\n");
        return 2;
    }
    const std::string dir = argv[1];
    const int order = atoi(argv[2]);
    int dtype, src, launches;
    unsigned num_blocks, P, H, D;
    {
        const std::vector<uint8_t> m = read_file(dir + "/meta.txt");
        const std::string s(m.begin(), m.end());
        if (sscanf(s.c_str(), "%d %d %u %u %u %u %d", &dtype, &src, &num_blocks, &P, &H, &D, &launches) != 7) return 2;
    }
    const std::vector<uint8_t> k0 = read_file(dir + "/pool_k.bin"), v0 = read_file(dir + "/pool_v.bin");
    const std::vector<uint8_t> ks0 = read_file(dir + "/pool_ks.bin", false), vs0 = read_file(dir + "/pool_vs.bin", false);
    uint8_t* k = exact_copy(k0);
    uint8_t* v = exact_copy(v0);
    uint8_t* ks = dtype == VSPEC_KV_INT4 ? exact_copy(ks0) : nullptr;
    uint8_t* vs = dtype == VSPEC_KV_INT4 ? exact_copy(vs0) : nullptr;
    for (int li = 0; li < launches; ++li) {
        const std::string pre = dir + "/L" + std::to_string(li);
        int mode;
        unsigned batch, n_new, max_blocks, n_items, rope_dim, max_pos;
        {
            const std::vector<uint8_t> m = read_file(pre + ".txt");
            const std::string s(m.begin(), m.end());
            if (sscanf(s.c_str(), "%d %u %u %u %u %u %u", &mode, &batch, &n_new, &max_blocks, &n_items, &rope_dim,
                       &max_pos) != 7)
                return 2;
        }
        uint8_t* tables = exact_copy(read_file(pre + "_tables.bin"));
        uint8_t* kn = exact_copy(read_file(pre + "_k.bin"));
        uint8_t* vn = exact_copy(read_file(pre + "_v.bin"));
        uint8_t *start = nullptr, *item = nullptr, *pos = nullptr, *ctx = nullptr, *cs = nullptr, *sn = nullptr;
        AppendParams p = {};
        p.k = k;
        p.v = v;
        p.ks = (uint16_t*)ks;
        p.vs = (uint16_t*)vs;
        p.kf = nullptr;  // int4 clamp flags need the wave's lanes: covered on the GPU
        p.block_tables = (const int32_t*)tables;
        if (mode == 0) {
            start = exact_copy(read_file(pre + "_start.bin"));
            p.start_pos = (const int32_t*)start;
        } else if (mode == 1) {
            item = exact_copy(read_file(pre + "_item.bin"));
            pos = exact_copy(read_file(pre + "_pos.bin"));
            p.token_item = (const int32_t*)item;
            p.token_pos = (const int32_t*)pos;
            p.n_items = n_items;
        } else {
            ctx = exact_copy(read_file(pre + "_ctx.bin"));
            p.ctx_lens = (const int32_t*)ctx;
        }
        if (rope_dim) {
            cs = exact_copy(read_file(pre + "_cos.bin"));
            sn = exact_copy(read_file(pre + "_sin.bin"));
            p.rope_cos = (const float*)cs;
            p.rope_sin = (const float*)sn;
            p.rope_dim = rope_dim;
            p.max_pos = max_pos;
        }
        p.k_new = kn;
        p.v_new = vn;
        p.batch = batch;
        p.n_new = n_new;
        p.hkv = H;
        p.head_dim = D;
        p.block_tokens = P;
        p.max_blocks = max_blocks;
        p.num_blocks = num_blocks;
        if (dtype == VSPEC_KV_F32) dispatch_src<VSPEC_KV_F32>(src, p, order);
        else if (dtype == VSPEC_KV_F16) dispatch_src<VSPEC_KV_F16>(src, p, order);
        else dispatch_src<VSPEC_KV_INT4>(src, p, order);
        for (uint8_t* b : {tables, kn, vn, start, item, pos, ctx, cs, sn}) free(b);
    }
    const std::string o = dir + "/out" + std::to_string(order);
    write_file(o + "_k.bin", k, k0.size());
    write_file(o + "_v.bin", v, v0.size());
    if (ks) write_file(o + "_ks.bin", ks, ks0.size());
    if (vs) write_file(o + "_vs.bin", vs, vs0.size());
    for (uint8_t* b : {k, v, ks, vs}) free(b);
    return 0;
}
