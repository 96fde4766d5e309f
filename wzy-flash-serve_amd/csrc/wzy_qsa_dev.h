// wzy_qsa_dev.h -- device helpers shared by the QSA decode kernels and the prefill kernels.
#pragma once
#include "wzy_device.h"
#include "wzy_qsa.h"

namespace wzy {

// RMSNorm(gamma) + NeoX RoPE (pairs i, i + n_rot/2) of one head vector p[0..hd) in place.
// 256 threads, thread i owns element i.
// reference: fused_head_norm_rope_multi (src/wzy_qsa_256k.cuh:50-82)
WZY_DEV void norm_rope(float* p, int hd, const float* gamma, const float* cos_tab, const float* sin_tab, int pos,
                       int n_rot, float eps, float* s_vals, float* s_red) {
    const int i = threadIdx.x;
    const float x = i < hd ? p[i] : 0.f;
    const float ss = block_sum<4>(x * x, s_red);
    const float sc = 1.0f / sqrtf(ss / (float) hd + eps);
    const float v = x * (sc * (i < hd ? gamma[i] : 0.f));
    if (i < hd) s_vals[i] = v;
    __syncthreads();
    const int half = n_rot / 2;
    if (i < hd) {
        float y = v;
        if (i < n_rot) {
            const int pr = i % half;
            const float c = cos_tab[(size_t) pos * half + pr], s = sin_tab[(size_t) pos * half + pr];
            const float a = s_vals[pr], d = s_vals[pr + half];
            y = (i < half) ? (a * c - d * s) : (a * s + d * c);
        }
        p[i] = y;
    }
    __syncthreads();
}

// Per-64 INT8 quantisation of element `threadIdx.x` (< hd) of KV head j's k and v rows into the
// store slot of position pos: scale = fp16(max|x| / 127) per 64-element group (one wave per group,
// every lane of the wave active), code = clamp(round(x / scale), +-127).
// reference: kv_append_int8_multi (src/wzy_qsa_256k.cuh:86-143)
WZY_DEV void qsa_kv_store(const QsaDims& dm, const QsaKv& kv, int pos, int j, float kval, float vval) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int hd = dm.hd, kvd = dm.kvh * dm.hd;
    const float kmax = wave_max(fabsf(kval)), vmax = wave_max(fabsf(vval));
    const uint16_t kh = f_to_h16(kmax / 127.0f), vh = f_to_h16(vmax / 127.0f);
    const float kdq = h16_to_f(kh), vdq = h16_to_f(vh);
    const int kqi = kdq > 0.f ? max(-127, min(127, rn_int(kval / kdq))) : 0;
    const int vqi = vdq > 0.f ? max(-127, min(127, rn_int(vval / vdq))) : 0;
    const size_t slot = qsa_kv_slot(pos, dm);
    kv.kq[slot * kvd + (size_t) j * hd + tid] = (int8_t) kqi;
    kv.vq[slot * kvd + (size_t) j * hd + tid] = (int8_t) vqi;
    if (lane == 0) {
        kv.ks[slot * (kvd / 64) + (size_t) j * (hd / 64) + w] = kh;
        kv.vs[slot * (kvd / 64) + (size_t) j * (hd / 64) + w] = vh;
    }
}

// Indexer key of one block (threads d < idim; 256 threads): the mean of the block's iblk cells,
// summed in cell order from cell(0) (cell(jj) is the fp16-rounded raw key value of cell jj for this
// thread's dimension), RMSNorm(ik_norm) over idim, NeoX RoPE at rope_pos.  Returns the key value of
// dimension d (0 for d >= idim).  reference: qsa_indexer_append_multi (src/wzy_qsa_256k.cuh:147-209)
template <class CellF>
WZY_DEV float idx_block_key(const QsaDims& dm, CellF cell, const float* ik_norm, const float* cos_tab,
                            const float* sin_tab, int rope_pos, float* s_vals, float* s_red) {
    const int d = threadIdx.x, D = dm.idim, B = dm.iblk, half = dm.n_rot / 2;
    float sum = 0.f;
    if (d < D) {
        sum = cell(0);
        for (int jj = 1; jj < B; ++jj) sum = sum + cell(jj);
    }
    const float mean = sum * (1.0f / (float) B);
    const float ss = block_sum<4>(mean * mean, s_red);
    const float sc = 1.0f / sqrtf(ss / (float) D + dm.eps);
    const float val = d < D ? sc * mean * ik_norm[d] : 0.f;
    s_vals[d] = val;
    __syncthreads();
    float y = val;
    if (d < D && d < dm.n_rot) {
        const int pr = d % half;
        const float c = cos_tab[(size_t) rope_pos * half + pr], s = sin_tab[(size_t) rope_pos * half + pr];
        const float x0 = s_vals[pr], z0 = s_vals[pr + half];
        y = (d < half) ? (x0 * c - z0 * s) : (x0 * s + z0 * c);
    }
    __syncthreads();
    return y;
}

}  // namespace wzy
