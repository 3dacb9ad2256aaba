/*
 * routing_oracle.c -- CPU restatement of the reference's MoE routing metadata
 * producers (kernels/moe-routing/* and the formulas of tests/test_moe.py).
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product path may link or call this
 * file; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * use it, and only as the checker.
 *
 * Plain scalar C following each reference routine step by step. How each one
 * is pinned is listed in oracle/oracle.py's header.
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);

/* moe-routing/moe_topk/kernel.cpp:89-205. Experts are scanned in index order;
 * a logit enters when it is greater than the current K-th value (initially
 * -FLT_MAX, so -inf never enters) and goes before the first held value it
 * exceeds (equal values keep scan order: lower expert first, -0 == +0).
 * One deliberate difference: NaN never enters (the reference's
 * `cval <= top[K-1]` test lets a NaN in at the last slot). Softmax:
 * expf(v_k - v_0) summed in k order, times 1 / sum. bits: row-major
 * [rows, ceil(E / 32)] (NULL: skipped). */
void orc_topk(const uint16_t* X, int64_t ldx, int64_t rows, int64_t E, int K, int softmax, uint16_t* Yv, int32_t* Yi,
              int64_t ldy, uint32_t* bits) {
    float top[64];
    int32_t ti[64];
    const int64_t nwords = (E + 31) / 32;
    for (int64_t r = 0; r < rows; ++r) {
        for (int k = 0; k < K; ++k) {
            top[k] = -FLT_MAX;
            ti[k] = -1;
        }
        for (int64_t e = 0; e < E; ++e) {
            const float c = orc_bf16_to_f32(X[r * ldx + e]);
            if (isnan(c) || c <= top[K - 1]) continue;
            int pos = K - 1;
            for (int k = 0; k < K; ++k)
                if (c > top[k]) {
                    pos = k;
                    break;
                }
            for (int k = K - 1; k > pos; --k) {
                top[k] = top[k - 1];
                ti[k] = ti[k - 1];
            }
            top[pos] = c;
            ti[pos] = (int32_t)e;
        }
        if (softmax) {
            const float mx = top[0];
            float sum = 0.0f;
            for (int k = 0; k < K; ++k) {
                top[k] = expf(top[k] - mx);
                sum += top[k];
            }
            const float inv = 1.0f / sum;
            for (int k = 0; k < K; ++k) top[k] *= inv;
        }
        for (int k = 0; k < K; ++k) {
            Yv[r * ldy + k] = orc_f32_to_bf16(top[k]);
            Yi[r * ldy + k] = ti[k];
        }
        if (bits) {
            for (int64_t w = 0; w < nwords; ++w) bits[r * nwords + w] = 0;
            for (int k = 0; k < K; ++k)
                if (ti[k] >= 0) bits[r * nwords + ti[k] / 32] |= 1u << (ti[k] % 32);
        }
    }
}

/* moe-routing/moe_bitmatrix/kernel.cpp:84-160 (and the fused form :168-204 over
 * all rows): B row-major [rows, nwords]; ret[e] = rows with bit e set;
 * partials (row-major [ceil(rows / 128), 32 * nwords], NULL: skipped) = the
 * count over the 128-row tiles before each tile. */
void orc_sum_bitmatrix_rows(const uint32_t* B, int64_t rows, int64_t nwords, uint32_t* ret, uint32_t* partials) {
    const int64_t E = 32 * nwords, ntiles = (rows + 127) / 128;
    for (int64_t e = 0; e < E; ++e) ret[e] = 0;
    for (int64_t t = 0; t < ntiles; ++t) {
        if (partials)
            for (int64_t e = 0; e < E; ++e) partials[t * E + e] = ret[e];
        for (int64_t r = t * 128; r < rows && r < (t + 1) * 128; ++r)
            for (int64_t e = 0; e < E; ++e)
                if ((B[r * nwords + e / 32] >> (e % 32)) & 1u) ret[e]++;
    }
}

/* moe-routing/moe_expt_data/kernel.cpp:25-106. mode 0: stage 1 (starts, and
 * 0xFFFFFFFF for tiles in [total, max_tiles)); mode 1: stage 1 + stage 2 (every
 * tile e | (i << 16)); mode 2: stage 1 + fused stage 2 (each expert's first
 * tile only). md entries not named by the mode keep the caller's contents;
 * no entry at or past max_tiles is written. */
void orc_expt_data(const int32_t* hist, int64_t E, int64_t max_tiles, int64_t n_gates, int log2, int mode,
                   int32_t* token_start, int32_t* tile_start, uint32_t* md) {
    const int64_t tile = (int64_t)1 << log2;
    int64_t tok = 0, til = 0;
    for (int64_t e = 0; e < E; ++e) {
        token_start[e] = (int32_t)tok;
        tile_start[e] = (int32_t)til;
        tok += hist[e];
        til += (hist[e] + tile - 1) / tile;
    }
    token_start[E] = (int32_t)n_gates;
    tile_start[E] = (int32_t)til;
    for (int64_t t = til; t < max_tiles; ++t) md[t] = 0xFFFFFFFFu;
    if (mode == 0) return;
    for (int64_t e = 0; e < E; ++e) {
        if (hist[e] <= 0) continue;
        const int64_t n = mode == 2 ? 1 : (hist[e] + tile - 1) / tile;
        for (int64_t i = 0; i < n; ++i)
            if (tile_start[e] + i < max_tiles) md[tile_start[e] + i] = (uint32_t)e | ((uint32_t)i << 16);
    }
}

/* moe-routing/moe_routing/kernel.cpp:78-205. Gates in 128-token blocks of
 * 128 * K gates; within a block the gates are stably sorted by expert and each
 * takes its exclusive run length r; pos = tokens_start[e] + partial[b, e] + r.
 * partial_offs (row-major [nblocks, E]) or, when NULL, the counts of the
 * earlier blocks. Ids outside [0, 1024) get scatter = -1 and no slot.
 * gate_scal / expt_scal may be NULL. */
void orc_compute_indx(const int32_t* indx, const uint16_t* expt_scal, int64_t n_gates, int K,
                      const int32_t* partial_offs, int64_t E, const int32_t* tokens_start, int32_t* gather,
                      int32_t* scatter, uint16_t* gate_scal) {
    const int64_t G = 128 * (int64_t)K;
    int64_t* carried = calloc(1024, sizeof(int64_t));
    int64_t* run = calloc(1024, sizeof(int64_t));
    for (int64_t b0 = 0; b0 < n_gates; b0 += G) {
        memset(run, 0, 1024 * sizeof(int64_t));
        for (int64_t g = b0; g < n_gates && g < b0 + G; ++g) {
            const int32_t e = indx[g];
            if (e < 0 || e >= 1024) {
                scatter[g] = -1;
                continue;
            }
            const int64_t base = partial_offs ? partial_offs[(b0 / G) * E + e] : carried[e];
            const int32_t pos = (int32_t)(tokens_start[e] + base + run[e]);
            run[e]++;
            scatter[g] = pos;
            gather[pos] = (int32_t)g;
            if (gate_scal) gate_scal[pos] = expt_scal[g];
        }
        for (int e = 0; e < 1024; ++e) carried[e] += run[e];
    }
    free(carried);
    free(run);
}

/* tests/test_moe.py:229-256 (the formula moe-routing/moe_align_block_size/
 * kernel.cpp:22-127 implements): per-expert counts, padded to block_size,
 * exclusive cumsum; ids placed in input order from cumsum[e]; padded slots =
 * numel; expert_ids[b] = e for the blocks of e. Ids outside [0, E) skipped.
 * sorted must hold numel + E * (bs - 1) entries; returns the total. */
int64_t orc_align_block_size(const int32_t* ids, int64_t numel, int64_t E, int64_t bs, int32_t* sorted,
                             int32_t* expert_ids, int32_t* cumsum) {
    int64_t* cnt = calloc((size_t)E, sizeof(int64_t));
    for (int64_t i = 0; i < numel; ++i)
        if (ids[i] >= 0 && ids[i] < E) cnt[ids[i]]++;
    cumsum[0] = 0;
    for (int64_t e = 0; e < E; ++e) cumsum[e + 1] = (int32_t)(cumsum[e] + (cnt[e] + bs - 1) / bs * bs);
    const int64_t total = cumsum[E];
    for (int64_t s = 0; s < total; ++s) sorted[s] = (int32_t)numel;
    memset(cnt, 0, (size_t)E * sizeof(int64_t));
    for (int64_t i = 0; i < numel; ++i) {
        const int32_t e = ids[i];
        if (e < 0 || e >= E) continue;
        sorted[cumsum[e] + cnt[e]++] = (int32_t)i;
    }
    for (int64_t e = 0; e < E; ++e)
        for (int64_t b = cumsum[e] / bs; b < cumsum[e + 1] / bs; ++b) expert_ids[b] = (int32_t)e;
    free(cnt);
    return total;
}
