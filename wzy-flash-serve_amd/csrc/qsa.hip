// qsa.hip -- QSA sparse-attention decode: per-row preparation and indexer block scores (gfx950).
//
//  qsa_prep   one launch, workgroup roles: q heads (RMSNorm + NeoX RoPE on the first n_rot dims),
//             kv heads (same on k, then per-64 INT8 quantisation of k and v into the KV store),
//             indexer q heads (RMSNorm + RoPE), and the indexer append (fp16-rounded key, 4-token
//             mean pooling, RMSNorm, RoPE at the block start, open-block placeholder).
//             reference: fused_head_norm_rope_multi, kv_append_int8_multi, qsa_indexer_append_multi
//             (src/wzy_qsa_256k.cuh:50-209)
//  qsa_score  score[b] = sum_h relu(fp16(q_h) . fp16(key_b)) for complete blocks (fp32 accumulate,
//             v_dot2_f32_f16), the open block against the fp32 placeholder key (+1e9 if partial).
//             Keys are stored as fp16 (the reference rounds its fp32 keys to fp16 when scoring), so
//             the scan reads 256 bytes per block.
//             reference: pf_qsa_block_scores_wmma, pf_qsa_tail_score_kernel (src/wzy_qsa_wmma.cuh:492-612)
// Selection and attention live in qsa_attn.hip.
#include "wzy_device.h"
#include "wzy_host.h"
#include "wzy_qsa.h"
#include "wzy_qsa_dev.h"

using namespace wzy;

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));


// ---------------------------------------------------------------------------------------------
// prep
// ---------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) qsa_prep_kernel(QsaPrepArgs a, int T) {
    __shared__ float s_vals[256];
    __shared__ float s_red[4];
    const QsaDims& dm = a.dm;
    const int wg = blockIdx.x, tid = threadIdx.x;
    const int base = *a.pos;
    const int hd = dm.hd, kvd = dm.kvh * dm.hd;

    if (wg < dm.qh) {
        if (!a.qg) return;
        for (int t = 0; t < T; ++t) {
            const int pos = base + t;
            if (pos < 0 || pos >= dm.ctx_max) continue;
            norm_rope(a.qg + (size_t) t * dm.qh * 2 * hd + (size_t) wg * 2 * hd, hd, a.q_norm, a.cos_tab, a.sin_tab,
                      pos, dm.n_rot, dm.eps, s_vals, s_red);
        }
        return;
    }
    if (wg < dm.qh + dm.kvh) {
        const int j = wg - dm.qh;
        for (int t = 0; t < T; ++t) {
            const int pos = base + t;
            if (pos < 0 || pos >= dm.ctx_max) continue;
            float* kp = a.kk + (size_t) t * kvd + (size_t) j * hd;
            norm_rope(kp, hd, a.k_norm, a.cos_tab, a.sin_tab, pos, dm.n_rot, dm.eps, s_vals, s_red);
            if (tid < hd) qsa_kv_store(dm, a.kv, pos, j, kp[tid], a.vv[(size_t) t * kvd + (size_t) j * hd + tid]);
            __syncthreads();
        }
        return;
    }
    if (wg < dm.qh + dm.kvh + dm.ih) {
        const int i = wg - dm.qh - dm.kvh;
        for (int t = 0; t < T; ++t) {
            const int pos = base + t;
            if (pos < 0 || pos >= dm.ctx_max) continue;
            norm_rope(a.q_idx + (size_t) t * dm.ih * dm.idim + (size_t) i * dm.idim, dm.idim, a.iq_norm, a.cos_tab,
                      a.sin_tab, pos, dm.n_rot, dm.eps, s_vals, s_red);
        }
        return;
    }
    if (dm.window > 0) return;                      // no indexer in window mode
    // indexer append (one workgroup, thread d owns key dim d)
    const int D = dm.idim, B = dm.iblk;
    const int d = tid;
    for (int t = 0; t < T; ++t) {
        const int pos = base + t;
        if (pos < 0 || pos >= dm.ctx_max) continue;
        const float incoming = d < D ? round_h16(a.idx_raw[(size_t) t * D + d]) : 0.f;
        const int slot = pos % B;
        if (d < D && slot < B - 1) a.ix.tail[slot * D + d] = incoming;
        const int b = pos / B;
        if (pos == 0 || slot == B - 1) {
            auto cell = [&](int jj) { return (pos == 0 || jj == B - 1) ? incoming : a.ix.tail[jj * D + d]; };
            const float y = idx_block_key(dm, cell, a.ik_norm, a.cos_tab, a.sin_tab, pos == 0 ? 0 : B * b, s_vals, s_red);
            if (d < D) {
                a.ix.pooled[(size_t) b * D + d] = f_to_h16(y);
                if (pos == 0) a.ix.dead[d] = y;
                else a.ix.pooled[(size_t) (b + 1) * D + d] = f_to_h16(a.ix.dead[d]);
            }
            __syncthreads();
        }
        if (a.ix.tail_snaps && d < D) {
            for (int jj = 0; jj < B - 1; ++jj)
                a.ix.tail_snaps[((size_t) t * (B - 1) + jj) * D + d] = a.ix.tail[jj * D + d];
            a.ix.dead_snaps[(size_t) t * D + d] = a.ix.dead[d];
            a.ix.pool_snaps[((size_t) t * 2 + 0) * D + d] = a.ix.pooled[(size_t) b * D + d];
            a.ix.pool_snaps[((size_t) t * 2 + 1) * D + d] = a.ix.pooled[(size_t) (b + 1) * D + d];
        }
    }
}

// ---------------------------------------------------------------------------------------------
// block scores
// ---------------------------------------------------------------------------------------------
constexpr int SC_BLOCKS_PER_WG = 64;

// Rows: a group of up to T rows per blockIdx.y (rows r0 .. r0+T-1 of a.rows, r0 = T * blockIdx.y).
template <int T>
__global__ void __launch_bounds__(256) qsa_score_kernel(QsaScoreArgs a) {
    __shared__ h2_t s_q[T][4][64];          // fp16 indexer queries, ih <= 4, idim = 128
    const QsaDims& dm = a.dm;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r0 = blockIdx.y * T, nrows = min(T, a.rows - r0);
    const int base = *a.pos + r0;
    const int D = dm.idim, B = dm.iblk, IH = dm.ih;
    const float* q_idx = a.q_idx + (size_t) r0 * IH * D;
    float* scores = a.scores + (size_t) r0 * a.max_b;
    const int n_kv_max = base + nrows;
    if (n_kv_max <= dm.topk) return;                    // short context: identity selection
    const int b0 = blockIdx.x * SC_BLOCKS_PER_WG;
    const bool tail_wg = blockIdx.x == 0;
    if (b0 >= n_kv_max / B && !tail_wg) return;

    for (int i = tid; i < T * IH * (D / 2); i += blockDim.x) {
        const int t = i / (IH * (D / 2)), r = i % (IH * (D / 2));
        const int h = r / (D / 2), k = r % (D / 2);
        h2_t v;
        v.x = v.y = (_Float16) 0.f;
        if (t < nrows) {
            const float* q = q_idx + (size_t) t * IH * D + (size_t) h * D + 2 * k;
            v.x = (_Float16) q[0];
            v.y = (_Float16) q[1];
        }
        s_q[t][h][k] = v;
    }
    __syncthreads();

    // complete blocks: 16 lanes per block (8 halves each), 4 blocks per wave-iteration; the keys of
    // all iterations are loaded before any is used
    const int li = lane & 15;
    constexpr int NIT = SC_BLOCKS_PER_WG / 16;
    const int b_lim = min(a.max_b, n_kv_max / B);
    uint4 kr[NIT];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int b = min(b0 + w * 16 + it * 4 + (lane >> 4), max(b_lim - 1, 0));
        kr[it] = *(const uint4*) (a.pooled + (size_t) b * D + 8 * li);
    }
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int b = b0 + w * 16 + it * 4 + (lane >> 4);
        if (b >= b_lim) continue;
        const uint4 kraw = kr[it];
        const h2_t k0 = __builtin_bit_cast(h2_t, kraw.x), k1 = __builtin_bit_cast(h2_t, kraw.y);
        const h2_t k2 = __builtin_bit_cast(h2_t, kraw.z), k3 = __builtin_bit_cast(h2_t, kraw.w);
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int n_kv = base + t + 1;
            float score = 0.f;
            for (int h = 0; h < IH; ++h) {
                float dd = 0.f;
                dd = __builtin_amdgcn_fdot2(s_q[t][h][4 * li + 0], k0, dd, false);
                dd = __builtin_amdgcn_fdot2(s_q[t][h][4 * li + 1], k1, dd, false);
                dd = __builtin_amdgcn_fdot2(s_q[t][h][4 * li + 2], k2, dd, false);
                dd = __builtin_amdgcn_fdot2(s_q[t][h][4 * li + 3], k3, dd, false);
                dd = sum16(dd);
                score += dd > 0.f ? dd : 0.f;
            }
            if (li == 0 && t < nrows && n_kv > dm.topk && b < n_kv / B) scores[(size_t) t * a.max_b + b] = score;
        }
    }
    // open block: fp32 dot with the placeholder key (wave t handles row t)
    if (tail_wg) {
        for (int t = w; t < nrows; t += 4) {
            const int n_kv = base + t + 1;
            const int nbid = n_kv / B;
            if (n_kv <= dm.topk || nbid >= a.max_b) continue;
            float score = 0.f;
            for (int h = 0; h < IH; ++h) {
                float p = 0.f;
                for (int k = lane; k < D; k += 64) p = fmaf(a.dead[k], q_idx[(size_t) t * IH * D + (size_t) h * D + k], p);
                p = wave_sum(p);
                score += p > 0.f ? p : 0.f;
            }
            if (n_kv % B != 0) score += 1e9f;
            if (lane == 0) scores[(size_t) t * a.max_b + nbid] = score;
        }
    }
}

// ---------------------------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------------------------
namespace wzy {

int qsa_check_dims(const QsaDims& dm) {
    WZY_REQUIRE(dm.hd == 256 && dm.kvh >= 1 && dm.qh % dm.kvh == 0 && dm.qh / dm.kvh <= 16,
                "qsa: head layout unsupported (hd 256, at most 16 q heads per kv head)");
    WZY_REQUIRE(dm.idim <= 128 && dm.idim % 8 == 0 && dm.ih <= 4 && dm.iblk >= 2, "qsa: indexer layout unsupported");
    WZY_REQUIRE(dm.n_rot % 2 == 0 && dm.n_rot <= dm.idim && dm.n_rot <= dm.hd, "qsa: bad n_rot");
    WZY_REQUIRE(dm.topk >= 1 && dm.ctx_max >= 1, "qsa: bad topk/ctx");
    if (dm.window > 0) {
        // a sliding window reads only the last `window` cells, so its ring may wrap
        WZY_REQUIRE(dm.ih == 0 && dm.sinks == 0 && dm.topk == dm.window && dm.window <= dm.ring_cap,
                    "qsa: window mode needs no indexer, no sinks, topk == window <= kv ring");
        return WZY_OK;
    }
    return qsa_check_ring(dm.ctx_max, dm.ring_cap, dm.sinks);
}

int qsa_check_ring(int ctx_max, int ring_cap, int sinks) {
    if (ring_cap == 0) {
        WZY_REQUIRE(sinks == 0, "qsa: kv_sinks %d given without a KV ring", sinks);
        return WZY_OK;
    }
    WZY_REQUIRE(ring_cap > 0 && sinks >= 0 && sinks < ring_cap, "qsa: bad KV ring (kv_ring %d, kv_sinks %d)",
                ring_cap, sinks);
    WZY_REQUIRE(ctx_max <= ring_cap,
                "qsa: a KV ring of %d cells cannot hold ctx_max %d; cells past the ring would read newer cells "
                "(use kv_ring 0: the full-context store)", ring_cap, ctx_max);
    return WZY_OK;
}

int launch_qsa_prep(const QsaPrepArgs& a, int T, hipStream_t st) {
    WZY_TRY(qsa_check_dims(a.dm));
    WZY_REQUIRE(T >= 1 && T <= WZY_MAX_W, "qsa_prep: T out of range");
    const int n_wg = a.dm.qh + a.dm.kvh + a.dm.ih + (a.dm.window > 0 ? 0 : 1);
    hipLaunchKernelGGL(qsa_prep_kernel, dim3(n_wg), dim3(256), 0, st, a, T);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

int launch_qsa_score(const QsaScoreArgs& a0, int T, hipStream_t st) {
    WZY_TRY(qsa_check_dims(a0.dm));
    WZY_REQUIRE(a0.dm.idim == 128, "qsa_score: indexer key width must be 128");
    WZY_REQUIRE(T >= 1 && T <= WZY_MAX_W, "qsa_score: T out of range");
    QsaScoreArgs a = a0;
    a.rows = T;
    const int grid = (a.max_b + SC_BLOCKS_PER_WG - 1) / SC_BLOCKS_PER_WG;
    switch (T) {
#define C_(TT) case TT: hipLaunchKernelGGL((qsa_score_kernel<TT>), dim3(grid), dim3(256), 0, st, a); break;
        C_(1) C_(2) C_(3) C_(4) C_(5) C_(6) C_(7)
        default: hipLaunchKernelGGL((qsa_score_kernel<8>), dim3(grid), dim3(256), 0, st, a); break;
#undef C_
    }
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

int launch_qsa_score_rows(const QsaScoreArgs& a0, int rows, hipStream_t st) {
    WZY_TRY(qsa_check_dims(a0.dm));
    WZY_REQUIRE(a0.dm.idim == 128, "qsa_score: indexer key width must be 128");
    WZY_REQUIRE(rows >= 1 && (rows + WZY_MAX_W - 1) / WZY_MAX_W <= 65535, "qsa_score: %d rows", rows);
    QsaScoreArgs a = a0;
    a.rows = rows;
    const int grid = (a.max_b + SC_BLOCKS_PER_WG - 1) / SC_BLOCKS_PER_WG;
    hipLaunchKernelGGL((qsa_score_kernel<WZY_MAX_W>), dim3(grid, (rows + WZY_MAX_W - 1) / WZY_MAX_W), dim3(256), 0, st,
                       a);
    WZY_LAUNCH_CHECK();
    return WZY_OK;
}

}  // namespace wzy

// ---------------------------------------------------------------------------------------------
// C ABI (device pointers; `pos` is a device int holding the position of row 0)
// ---------------------------------------------------------------------------------------------
static QsaDims dims_of(const wzy_qsa_dims* s) {
    QsaDims d;
    d.qh = s->qh; d.kvh = s->kvh; d.hd = s->hd; d.n_rot = s->n_rot;
    d.ih = s->idx_heads; d.idim = s->idx_dim; d.iblk = s->idx_blk; d.topk = s->idx_topk;
    d.ctx_max = s->ctx_max; d.ring_cap = s->kv_ring; d.sinks = s->kv_sinks; d.eps = s->eps;
    d.f16_above = s->attn_f16_above;
    return d;
}

extern "C" int wzy_qsa_prepare(const wzy_qsa_dims* dims, const int* pos, float* qg, float* kk, const float* vv,
                               float* q_idx, const float* idx_raw, const float* q_norm, const float* k_norm,
                               const float* iq_norm, const float* ik_norm, const float* cos_tab, const float* sin_tab,
                               int8_t* kq, uint16_t* ks, int8_t* vq, uint16_t* vs, float* idx_tail, float* idx_dead,
                               uint16_t* idx_pooled, int T, void* stream) {
    WZY_REQUIRE(dims && pos && qg && kk && vv && q_idx && idx_raw && kq && ks && vq && vs && idx_tail && idx_dead &&
                    idx_pooled && cos_tab && sin_tab && q_norm && k_norm && iq_norm && ik_norm,
                "wzy_qsa_prepare: null pointer");
    QsaPrepArgs a{};
    a.dm = dims_of(dims);
    a.pos = pos; a.qg = qg; a.kk = kk; a.vv = vv; a.q_idx = q_idx; a.idx_raw = idx_raw;
    a.q_norm = q_norm; a.k_norm = k_norm; a.iq_norm = iq_norm; a.ik_norm = ik_norm;
    a.cos_tab = cos_tab; a.sin_tab = sin_tab;
    a.kv = QsaKv{kq, ks, vq, vs};
    a.ix.tail = idx_tail; a.ix.dead = idx_dead; a.ix.pooled = idx_pooled;
    return launch_qsa_prep(a, T, as_stream(stream));
}

extern "C" int wzy_qsa_select(const wzy_qsa_dims* dims, const int* pos, const uint16_t* idx_pooled,
                              const float* idx_dead, const float* q_idx, float* scores, int max_b, int* sel_ids,
                              int* sel_cnt, int T, void* stream) {
    WZY_REQUIRE(dims && pos && idx_pooled && idx_dead && q_idx && scores && sel_ids && sel_cnt,
                "wzy_qsa_select: null pointer");
    QsaScoreArgs s{};
    s.dm = dims_of(dims);
    WZY_REQUIRE(max_b >= dims->ctx_max / dims->idx_blk + 1, "wzy_qsa_select: max_b too small");
    s.pos = pos; s.pooled = idx_pooled; s.dead = idx_dead; s.q_idx = q_idx; s.scores = scores; s.max_b = max_b;
    hipStream_t st = as_stream(stream);
    WZY_TRY(launch_qsa_score(s, T, st));
    return launch_qsa_topk(s.dm, pos, scores, max_b, sel_ids, sel_cnt, T, st);
}

extern "C" int wzy_qsa_topk(const wzy_qsa_dims* dims, const int* pos, const float* scores, int max_b, int* sel_ids,
                            int* sel_cnt, int T, void* stream) {
    WZY_REQUIRE(dims && pos && scores && sel_ids && sel_cnt, "wzy_qsa_topk: null pointer");
    WZY_REQUIRE(max_b >= dims->ctx_max / dims->idx_blk + 1, "wzy_qsa_topk: max_b too small");
    return launch_qsa_topk(dims_of(dims), pos, scores, max_b, sel_ids, sel_cnt, T, as_stream(stream));
}

extern "C" size_t wzy_qsa_attend_workspace_bytes(const wzy_qsa_dims* dims, int T) {
    const QsaDims d = dims_of(dims);
    const size_t pf = qsa_attn_part_floats(d, T);
    return (pf + pf / d.hd * 2) * sizeof(float) + 512;
}

extern "C" int wzy_qsa_attend(const wzy_qsa_dims* dims, const int* pos, const float* qg, const int8_t* kq,
                              const uint16_t* ks, const int8_t* vq, const uint16_t* vs, const int* sel_ids, float* out,
                              void* workspace, size_t workspace_bytes, int T, void* stream) {
    WZY_REQUIRE(dims && pos && qg && kq && ks && vq && vs && sel_ids && out && workspace,
                "wzy_qsa_attend: null pointer");
    WZY_REQUIRE(workspace_bytes >= wzy_qsa_attend_workspace_bytes(dims, T), "wzy_qsa_attend: workspace too small");
    QsaAttnArgs a{};
    a.dm = dims_of(dims);
    a.pos = pos; a.qg = qg; a.kv = QsaKv{(int8_t*) kq, (uint16_t*) ks, (int8_t*) vq, (uint16_t*) vs};
    a.sel_ids = sel_ids; a.out = out;
    const size_t pf = qsa_attn_part_floats(a.dm, T);
    a.part = (float*) workspace;
    a.part_ml = a.part + pf;
    return launch_qsa_attn(a, T, as_stream(stream));
}
