// decode.hip -- split-K decode attention over a GQA fp16 KV cache (gfx950).
//
// Work decomposition: one 64-lane workgroup per (split, kv_head, sequence).
// A split is a page-aligned chunk of `chunk` tokens (a multiple of 64); the
// workgroup serves all G = Hq/Hkv query heads of its KV head, so every K/V
// byte is read from HBM exactly once (the reference re-reads each KV row once
// per query head, src/cuda/decode_attention_split.cu:40-49).
//
// Per 64-token iteration (4 pages of 16 tokens):
//   QK^T  on MFMA: v_mfma_f32_16x16x32_f16 with B = K^T (lane l holds 16 B of
//         token (page t, slot l%16) at dims 32c + 8(l/16)) and A = Q (row r
//         holds head r % CG).  Accumulator tile t then holds, in lane l,
//         scores of token (t, l%16) for heads 4(l/16)+e (mod CG); lane l keeps
//         the tile that belongs to it, so the 64 lanes hold 64 tokens x CG
//         heads with no redundancy.  K loads are 16 B per lane, 64 B
//         contiguous per row, full 64 B sectors.
//   softmax in fp32, log2 domain (scores pre-scaled by log2(e)/sqrt(D)),
//         wave64 DPP row reductions + 2 cross-row swizzles for the running
//         max; p and the rescale factors go through 2 KiB of LDS.
//   PV    on VALU: lane l owns 8 dims of one token per V load (16 B, a wave
//         load covers whole 256 B rows, 1 KiB contiguous), so V is read in
//         address order; fp32 FMAs, one accumulator set per lane row.
// Loads for iteration i+1 are issued while iteration i computes (K after the
// QK MFMAs retire their operands, V after PV).
//
// Split merge: each non-final split stores (m, l, o[D]) in fp32; the
// last-arriving workgroup of a (sequence, kv_head) -- found with a ticket
// counter in the workspace -- merges by log-sum-exp and writes fp16 output,
// so a decode is a single kernel launch.  Counters are returned to zero by
// the merging workgroup.
//
// Roofline: HBM-bound; algorithmic bytes per (token, kv_head) are 4*D
// (K + V fp16) plus the q read and output write per query head.
#include "kvhp_internal.h"

#include <cmath>
#include <mutex>
#include <vector>

namespace kvhp {

namespace {

constexpr int kMaxSplits = 1024;

struct KVDev {
    const f16* data;
    int64_t stride_b, stride_h, stride_s, stride_d;
    const int32_t* bt;
    int32_t max_pages;
    int32_t page_size;
    int32_t num_pages;
};

struct DecodeArgs {
    const f16* q;          // [B][Hq][D]
    KVDev k, v;
    const int32_t* seq_lens;
    f16* out;              // [B][Hq][D]
    float* ws_o;           // [B*Hq][nsplit][D]
    float* ws_ml;          // [B*Hq][nsplit][2]  (max in log2 units, sum)
    uint32_t* tickets;     // [B*Hkv]
    int Hq, Hkv;
    int chunk;             // tokens per split, multiple of 64
    int nsplit;            // split slots in the workspace
    int cap;               // tokens addressable per sequence (= nsplit*chunk)
    int fixed_len;         // length of every sequence when seq_lens == nullptr
    float scale_log2;      // log2(e) / sqrt(D)
};

__device__ __forceinline__ int seq_len_of(const DecodeArgs& a, int b) {
    return a.seq_lens ? a.seq_lens[b] : a.fixed_len;
}

template <bool PAGED>
__device__ __forceinline__ const f16* page_base(const f16* base, const int32_t* bt_row,
                                                int64_t ss, int page_idx,
                                                int num_pages) {
    if constexpr (PAGED) {
        int pid = bt_row[page_idx];
        pid = pid < 0 ? 0 : (pid >= num_pages ? num_pages - 1 : pid);
        return base + (int64_t)pid * kPage * ss;
    } else {
        return base + (int64_t)page_idx * kPage * ss;
    }
}

template <int D, int G, bool PAGED>
__global__ void __launch_bounds__(kWave)
decode_splitk_kernel(const DecodeArgs a) {
    constexpr int CG = G <= 4 ? 4 : (G <= 8 ? 8 : 16);  // heads per MFMA row set
    constexpr int NC = D / 32;       // MFMA k-chunks over head_dim
    constexpr int LPR = D / 8;       // lanes per V row (16 B each)
    constexpr int RPL = kWave / LPR; // V rows per wave load
    constexpr int NVL = 64 / RPL;    // V loads per 64-token iteration
    constexpr int R = CG / 4;        // score rounds (4 heads per lane each)
    constexpr int TPR = 4 / R;       // 16-token tiles per round
    constexpr int GQ = (G + 3) / 4;  // float4 groups of p read per token

    __shared__ floatx4 p_lds[2][64][CG / 4];
    __shared__ float alpha_lds[2][CG];
    __shared__ float m_lds[CG];
    __shared__ float w_lds[kMaxSplits];
    __shared__ uint32_t ticket_lds;

    const int lane = threadIdx.x;
    const int g = lane >> 4;
    const int col = lane & 15;
    const int split = blockIdx.x;
    const int kvh = blockIdx.y;
    const int b = blockIdx.z;
    const int64_t row0 = (int64_t)b * a.Hq + (int64_t)kvh * G;  // first q row

    int L = seq_len_of(a, b);
    if (L > a.cap) L = a.cap;
    if (L <= 0) {
        if (split == 0) {
            const half8 z = {};
            for (int i = lane; i < G * LPR; i += kWave)
                store_half8(a.out + (row0 + i / LPR) * D + 8 * (i % LPR), z);
        }
        return;
    }
    const int nsb = (L + a.chunk - 1) / a.chunk;
    if (split >= nsb) return;
    const int t_begin = split * a.chunk;
    const int t_end = min(L, t_begin + a.chunk);
    const int n_iter = (t_end - t_begin + 63) >> 6;
    const int last_tok = L - 1;
    const int last_pi = last_tok >> 4;

    const int64_t ssk = a.k.stride_s, ssv = a.v.stride_s;
    const f16* kbase;
    const f16* vbase;
    const int32_t* btk = nullptr;
    const int32_t* btv = nullptr;
    if constexpr (PAGED) {
        kbase = a.k.data + kvh * a.k.stride_h;
        vbase = a.v.data + kvh * a.v.stride_h;
        btk = a.k.bt + (int64_t)b * a.k.max_pages;
        btv = a.v.bt + (int64_t)b * a.v.max_pages;
    } else {
        kbase = a.k.data + b * a.k.stride_b + kvh * a.k.stride_h;
        vbase = a.v.data + b * a.v.stride_b + kvh * a.v.stride_h;
    }
    const f16* klast = page_base<PAGED>(kbase, btk, ssk, last_pi, a.k.num_pages) +
                       (last_tok & 15) * ssk;
    const f16* vlast = page_base<PAGED>(vbase, btv, ssv, last_pi, a.v.num_pages) +
                       (last_tok & 15) * ssv;

    // A operand: lane l holds q[head (l%16) % CG][dims 32c + 8(l/16) .. +8].
    half8 qa[NC];
    {
        const int hq = col % CG;
        if (hq < G) {
            const f16* qp = a.q + (row0 + hq) * D + 8 * g;
#pragma unroll
            for (int c = 0; c < NC; ++c) qa[c] = load_half8(qp + 32 * c);
        } else {
#pragma unroll
            for (int c = 0; c < NC; ++c) qa[c] = half8{};
        }
    }

    half8 kreg[4][NC];
    half8 vreg[NVL];
    const int vrow = lane / LPR;
    const int vdim = 8 * (lane % LPR);

    auto load_k = [&](int T0) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int pi = min((T0 >> 4) + t, last_pi);
            const f16* pg = page_base<PAGED>(kbase, btk, ssk, pi, a.k.num_pages);
            const int tok = T0 + 16 * t + col;
            const f16* rp = (tok <= last_tok) ? pg + col * ssk : klast;
#pragma unroll
            for (int c = 0; c < NC; ++c) kreg[t][c] = load_half8(rp + 32 * c + 8 * g);
        }
    };
    auto load_v = [&](int T0) {
#pragma unroll
        for (int j = 0; j < NVL; ++j) {
            const int t = (RPL * j) >> 4;
            const int slot = ((RPL * j) & 15) + vrow;
            const int pi = min((T0 >> 4) + t, last_pi);
            const f16* pg = page_base<PAGED>(vbase, btv, ssv, pi, a.v.num_pages);
            const int tok = T0 + RPL * j + vrow;
            const f16* rp = (tok <= last_tok) ? pg + slot * ssv : vlast;
            vreg[j] = load_half8(rp + vdim);
        }
    };

    float m_run[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) m_run[e] = -1e30f;
    float acc[G][8];
    float lsum[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        lsum[h] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
    }

    load_k(t_begin);
    load_v(t_begin);

    for (int it = 0; it < n_iter; ++it) {
        const int T0 = t_begin + 64 * it;
        const int par = it & 1;

        // ---- S = Q K^T on MFMA, one accumulator per 16-token tile.
        floatx4 C[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            C[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NC; ++c)
                C[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[c], kreg[t][c], C[t], 0, 0, 0);
        }
        if (it + 1 < n_iter) load_k(T0 + 64);

        // ---- scores of the lane's own tokens (heads 4*(g%R)+e).
        float s[R][4];
        int tile_of[R];
#pragma unroll
        for (int rr = 0; rr < R; ++rr) {
            const int sub = g / R;
            floatx4 sel = C[rr * TPR];
#pragma unroll
            for (int u = 1; u < TPR; ++u)
                if (sub == u) sel = C[rr * TPR + u];
            const int tile = rr * TPR + sub;
            tile_of[rr] = tile;
            const bool ok = T0 + 16 * tile + col < t_end;
#pragma unroll
            for (int e = 0; e < 4; ++e) s[rr][e] = ok ? sel[e] * a.scale_log2 : -INFINITY;
        }

        // ---- running max per head over the wave, rescale factor.
        float alpha[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float mt = s[0][e];
#pragma unroll
            for (int rr = 1; rr < R; ++rr) mt = fmaxf(mt, s[rr][e]);
            mt = row16_max(mt);
            if constexpr (R == 1) mt = fmaxf(mt, __shfl_xor(mt, 16));
            if constexpr (R <= 2) mt = fmaxf(mt, __shfl_xor(mt, 32));
            const float mn = fmaxf(m_run[e], mt);
            alpha[e] = fast_exp2(m_run[e] - mn);
            m_run[e] = mn;
        }
#pragma unroll
        for (int rr = 0; rr < R; ++rr) {
            floatx4 pv;
#pragma unroll
            for (int e = 0; e < 4; ++e) pv[e] = fast_exp2(s[rr][e] - m_run[e]);
            p_lds[par][16 * tile_of[rr] + col][g % R] = pv;
        }
        if (col == 0 && g < R) {
#pragma unroll
            for (int e = 0; e < 4; ++e) alpha_lds[par][4 * g + e] = alpha[e];
        }
        __syncthreads();

        // ---- O += P V on VALU in the V-row layout.
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float al = alpha_lds[par][h];
            lsum[h] *= al;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[h][e] *= al;
        }
#pragma unroll
        for (int j = 0; j < NVL; ++j) {
            const int tok = RPL * j + vrow;
            float pw[GQ * 4];
#pragma unroll
            for (int u = 0; u < GQ; ++u) {
                const floatx4 t4 = p_lds[par][tok][u];
                pw[4 * u + 0] = t4[0];
                pw[4 * u + 1] = t4[1];
                pw[4 * u + 2] = t4[2];
                pw[4 * u + 3] = t4[3];
            }
            float vf[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) vf[e] = static_cast<float>(vreg[j][e]);
#pragma unroll
            for (int h = 0; h < G; ++h) {
                lsum[h] += pw[h];
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[h][e] = fmaf(pw[h], vf[e], acc[h][e]);
            }
        }
        if (it + 1 < n_iter) load_v(T0 + 64);
    }

    // ---- combine the V-row partial sums (lanes with equal lane % LPR).
#pragma unroll
    for (int off = LPR; off < kWave; off <<= 1) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            lsum[h] += __shfl_xor(lsum[h], off);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[h][e] += __shfl_xor(acc[h][e], off);
        }
    }
    if (col == 0 && g < R) {
#pragma unroll
        for (int e = 0; e < 4; ++e) m_lds[4 * g + e] = m_run[e];
    }
    __syncthreads();

    if (nsb == 1) {
        if (lane < LPR) {
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float inv = lsum[h] > 0.f ? 1.f / lsum[h] : 0.f;
                half8 o;
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = static_cast<f16>(acc[h][e] * inv);
                store_half8(a.out + (row0 + h) * D + 8 * lane, o);
            }
        }
        return;
    }

    // ---- split partial, then the last workgroup of this (b, kv_head) merges.
    if (lane < LPR) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float* po = a.ws_o + ((row0 + h) * a.nsplit + split) * D + 8 * lane;
            *reinterpret_cast<floatx4*>(po) = floatx4{acc[h][0], acc[h][1], acc[h][2], acc[h][3]};
            *reinterpret_cast<floatx4*>(po + 4) = floatx4{acc[h][4], acc[h][5], acc[h][6], acc[h][7]};
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float* pm = a.ws_ml + ((row0 + h) * a.nsplit + split) * 2;
            pm[0] = m_lds[h];
            pm[1] = lsum[h];
        }
    }
    __threadfence();
    if (lane == 0) ticket_lds = atomicAdd(a.tickets + (int64_t)b * a.Hkv + kvh, 1u);
    __syncthreads();
    if (ticket_lds != static_cast<uint32_t>(nsb - 1)) return;
    __threadfence();

    constexpr int DPL = D / kWave;  // output dims per lane in the merge
    for (int h = 0; h < G; ++h) {
        const int64_t base = (row0 + h) * a.nsplit;
        float mx = -INFINITY;
        for (int j = lane; j < nsb; j += kWave) mx = fmaxf(mx, a.ws_ml[(base + j) * 2]);
        mx = wave_max(mx);
        float ls = 0.f;
        for (int j = lane; j < nsb; j += kWave) {
            const float w = fast_exp2(a.ws_ml[(base + j) * 2] - mx);
            w_lds[j] = w;
            ls += w * a.ws_ml[(base + j) * 2 + 1];
        }
        ls = wave_sum(ls);
        __syncthreads();
        const float inv = ls > 0.f ? 1.f / ls : 0.f;
        float o[DPL];
#pragma unroll
        for (int u = 0; u < DPL; ++u) o[u] = 0.f;
        for (int j = 0; j < nsb; ++j) {
            const float w = w_lds[j];
            const float* po = a.ws_o + (base + j) * D + DPL * lane;
#pragma unroll
            for (int u = 0; u < DPL; ++u) o[u] = fmaf(w, po[u], o[u]);
        }
#pragma unroll
        for (int u = 0; u < DPL; ++u)
            a.out[(row0 + h) * D + DPL * lane + u] = static_cast<f16>(o[u] * inv);
        __syncthreads();
    }
    if (lane == 0) atomicExch(a.tickets + (int64_t)b * a.Hkv + kvh, 0u);
}

// Any head_dim <= 256, any group size, any page size, any strides: one wave
// per (q_head, sequence), one pass over the keys with an online softmax.
// Serves shapes outside the fast kernel's template set.
template <bool PAGED>
__global__ void __launch_bounds__(kWave)
decode_generic_kernel(const DecodeArgs a, int D, int G) {
    const int lane = threadIdx.x;
    const int qh = blockIdx.x;
    const int b = blockIdx.y;
    const int kvh = qh / G;
    const int64_t row = (int64_t)b * a.Hq + qh;
    int L = seq_len_of(a, b);
    if (L > a.cap) L = a.cap;
    f16* o = a.out + row * D;
    if (L <= 0) {
        for (int d = lane; d < D; d += kWave) o[d] = f16(0);
        return;
    }
    float qv[4], acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int d = lane + kWave * i;
        qv[i] = d < D ? static_cast<float>(a.q[row * D + d]) : 0.f;
        acc[i] = 0.f;
    }
    float m = -1e30f, l = 0.f;
    for (int t = 0; t < L; ++t) {
        const f16* kr;
        const f16* vr;
        if constexpr (PAGED) {
            const int ps = a.k.page_size;
            int pk = a.k.bt[(int64_t)b * a.k.max_pages + t / ps];
            int pv = a.v.bt[(int64_t)b * a.v.max_pages + t / ps];
            pk = pk < 0 ? 0 : (pk >= a.k.num_pages ? a.k.num_pages - 1 : pk);
            pv = pv < 0 ? 0 : (pv >= a.v.num_pages ? a.v.num_pages - 1 : pv);
            kr = a.k.data + kvh * a.k.stride_h + ((int64_t)pk * ps + t % ps) * a.k.stride_s;
            vr = a.v.data + kvh * a.v.stride_h + ((int64_t)pv * ps + t % ps) * a.v.stride_s;
        } else {
            kr = a.k.data + b * a.k.stride_b + kvh * a.k.stride_h + t * a.k.stride_s;
            vr = a.v.data + b * a.v.stride_b + kvh * a.v.stride_h + t * a.v.stride_s;
        }
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = lane + kWave * i;
            if (d < D) dot = fmaf(qv[i], static_cast<float>(kr[d * a.k.stride_d]), dot);
        }
        dot = wave_sum(dot);
        const float sc = dot * a.scale_log2;
        const float mn = fmaxf(m, sc);
        const float al = fast_exp2(m - mn);
        const float p = fast_exp2(sc - mn);
        l = l * al + p;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = lane + kWave * i;
            const float vv = d < D ? static_cast<float>(vr[d * a.v.stride_d]) : 0.f;
            acc[i] = fmaf(p, vv, acc[i] * al);
        }
        m = mn;
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int d = lane + kWave * i;
        if (d < D) o[d] = static_cast<f16>(acc[i] * inv);
    }
}

// ------------------------------------------------------------- host side --
struct Plan {
    int nsplit;
    int chunk;
};

Plan make_plan(int batch, int num_kv_heads, int max_seq_len, int num_splits) {
    Plan p;
    if (max_seq_len < 1) max_seq_len = 1;
    const int max_by_chunk = (max_seq_len + 63) / 64;  // chunks of >= 64 tokens
    int s = num_splits;
    if (s <= 0) {
        // Aim for ~16 resident waves per CU over 256 CUs, no chunk below 64.
        const int64_t units = (int64_t)batch * num_kv_heads;
        const int64_t target = 4096;
        s = static_cast<int>((target + units - 1) / units);
    }
    if (s > max_by_chunk) s = max_by_chunk;
    if (s < 1) s = 1;
    int chunk = (max_seq_len + s - 1) / s;
    chunk = (chunk + 63) / 64 * 64;
    int n = (max_seq_len + chunk - 1) / chunk;
    while (n > kMaxSplits) {
        chunk += 64;
        n = (max_seq_len + chunk - 1) / chunk;
    }
    p.nsplit = n;
    p.chunk = chunk;
    return p;
}

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

size_t workspace_bytes_for(int batch, int hq, int hkv, int d, const Plan& p) {
    if (p.nsplit <= 1) return 0;
    const size_t tickets = align256(sizeof(uint32_t) * (size_t)batch * hkv);
    const size_t o = align256(sizeof(float) * (size_t)batch * hq * p.nsplit * d);
    const size_t ml = align256(sizeof(float) * (size_t)batch * hq * p.nsplit * 2);
    return tickets + o + ml;
}

// Library-owned per-device workspace used when the caller passes none.
struct DeviceWorkspace {
    void* ptr = nullptr;
    size_t bytes = 0;
};
std::mutex g_ws_mutex;
std::vector<DeviceWorkspace> g_ws;

int internal_workspace(size_t need, void** out) {
    int dev = 0;
    KVHP_HIP(hipGetDevice(&dev), "hipGetDevice");
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    if ((int)g_ws.size() <= dev) g_ws.resize(dev + 1);
    DeviceWorkspace& w = g_ws[dev];
    if (w.bytes < need) {
        if (w.ptr) KVHP_HIP(hipFree(w.ptr), "hipFree(workspace)");
        w.ptr = nullptr;
        w.bytes = 0;
        size_t grow = need < (size_t(1) << 20) ? (size_t(1) << 20) : need;
        KVHP_HIP(hipMalloc(&w.ptr, grow), "hipMalloc(workspace)");
        KVHP_HIP(hipMemset(w.ptr, 0, grow), "hipMemset(workspace)");
        w.bytes = grow;
    }
    *out = w.ptr;
    return KVHP_OK;
}

KVDev to_dev(const kvhp_kv_view& v) {
    KVDev d;
    d.data = static_cast<const f16*>(v.data);
    d.stride_b = v.stride_b;
    d.stride_h = v.stride_h;
    d.stride_s = v.stride_s;
    d.stride_d = v.stride_d;
    d.bt = v.block_table;
    d.max_pages = v.max_pages;
    d.page_size = v.page_size;
    d.num_pages = v.num_pages;
    return d;
}

bool view_fast_ok(const kvhp_kv_view& v) {
    if (v.stride_d != 1 || v.stride_s % 8 != 0 || !aligned16(v.data)) return false;
    if (v.block_table) return v.page_size == kPage && v.stride_h % 8 == 0;
    return v.stride_b % 8 == 0 && v.stride_h % 8 == 0;
}

template <int D, int G>
void launch_fast(const DecodeArgs& a, dim3 grid, bool paged, hipStream_t s) {
    if (paged)
        hipLaunchKernelGGL((decode_splitk_kernel<D, G, true>), grid, dim3(kWave), 0, s, a);
    else
        hipLaunchKernelGGL((decode_splitk_kernel<D, G, false>), grid, dim3(kWave), 0, s, a);
}

template <int D>
bool dispatch_g(int G, const DecodeArgs& a, dim3 grid, bool paged, hipStream_t s) {
    switch (G) {
        case 1: launch_fast<D, 1>(a, grid, paged, s); return true;
        case 2: launch_fast<D, 2>(a, grid, paged, s); return true;
        case 3: launch_fast<D, 3>(a, grid, paged, s); return true;
        case 4: launch_fast<D, 4>(a, grid, paged, s); return true;
        case 5: launch_fast<D, 5>(a, grid, paged, s); return true;
        case 6: launch_fast<D, 6>(a, grid, paged, s); return true;
        case 7: launch_fast<D, 7>(a, grid, paged, s); return true;
        case 8: launch_fast<D, 8>(a, grid, paged, s); return true;
        case 16: launch_fast<D, 16>(a, grid, paged, s); return true;
        default: return false;
    }
}

bool fast_group(int G) { return (G >= 1 && G <= 8) || G == 16; }

int validate_view(const kvhp_kv_view* v, const char* name) {
    KVHP_REQUIRE(v && v->data, KVHP_ERR_INVALID, "decode_attention: %s view is null", name);
    if (v->block_table) {
        KVHP_REQUIRE(v->max_pages > 0 && v->num_pages > 0 && v->page_size > 0,
                     KVHP_ERR_INVALID,
                     "decode_attention: %s paged view needs max_pages/num_pages/page_size > 0",
                     name);
    }
    return KVHP_OK;
}

}  // namespace

// seq_lens == nullptr: every sequence has length fixed_len (host value).
int decode_attention_impl(const void* q, const kvhp_kv_view* kv, const kvhp_kv_view* vv,
                          const int32_t* seq_lens, int fixed_len, void* out, int batch,
                          int hq, int hkv, int d, int max_seq_len, int num_splits,
                          void* workspace, size_t workspace_bytes, hipStream_t s) {
    if (batch <= 0 || max_seq_len <= 0) return KVHP_OK;
    KVHP_REQUIRE(q && out, KVHP_ERR_INVALID, "decode_attention: null pointer");
    KVHP_REQUIRE(hq > 0 && hkv > 0 && hq % hkv == 0, KVHP_ERR_INVALID,
                 "decode_attention: num_q_heads=%d must be a positive multiple of num_kv_heads=%d",
                 hq, hkv);
    KVHP_REQUIRE(d > 0 && d <= 256, KVHP_ERR_UNSUPPORTED,
                 "decode_attention: head_dim=%d outside 1..256", d);
    int rc = validate_view(kv, "K");
    if (rc) return rc;
    rc = validate_view(vv, "V");
    if (rc) return rc;
    KVHP_REQUIRE((kv->block_table == nullptr) == (vv->block_table == nullptr),
                 KVHP_ERR_INVALID, "decode_attention: K and V views must both be paged or both strided");
    const bool paged = kv->block_table != nullptr;
    const int G = hq / hkv;

    DecodeArgs a;
    a.q = static_cast<const f16*>(q);
    a.k = to_dev(*kv);
    a.v = to_dev(*vv);
    a.seq_lens = seq_lens;
    a.fixed_len = fixed_len;
    a.out = static_cast<f16*>(out);
    a.Hq = hq;
    a.Hkv = hkv;
    a.scale_log2 = 1.4426950408889634f / std::sqrt(static_cast<float>(d));

    const bool fast = (d == 64 || d == 128) && fast_group(G) && view_fast_ok(*kv) &&
                      view_fast_ok(*vv) && aligned16(q) && aligned16(out);
    if (!fast) {
        // Single pass: every sequence fully, no workspace.
        a.ws_o = nullptr;
        a.ws_ml = nullptr;
        a.tickets = nullptr;
        a.chunk = max_seq_len;
        a.nsplit = 1;
        a.cap = max_seq_len;
        if (paged) a.cap = min(a.cap, min(kv->max_pages * kv->page_size,
                                          vv->max_pages * vv->page_size));
        dim3 grid(hq, batch);
        if (paged)
            hipLaunchKernelGGL(decode_generic_kernel<true>, grid, dim3(kWave), 0, s, a, d, G);
        else
            hipLaunchKernelGGL(decode_generic_kernel<false>, grid, dim3(kWave), 0, s, a, d, G);
        return check_launch("decode_attention(generic)");
    }

    const Plan plan = make_plan(batch, hkv, max_seq_len, num_splits);
    a.chunk = plan.chunk;
    a.nsplit = plan.nsplit;
    a.cap = plan.nsplit * plan.chunk;
    if (a.cap > max_seq_len) a.cap = max_seq_len;
    // Never address block-table columns past max_pages.
    if (paged) a.cap = min(a.cap, min(kv->max_pages, vv->max_pages) * kPage);
    const size_t need = workspace_bytes_for(batch, hq, hkv, d, plan);
    a.ws_o = nullptr;
    a.ws_ml = nullptr;
    a.tickets = nullptr;
    if (need > 0) {
        void* ws = workspace;
        if (!ws) {
            rc = internal_workspace(need, &ws);
            if (rc) return rc;
        } else {
            KVHP_REQUIRE(workspace_bytes >= need, KVHP_ERR_WORKSPACE,
                         "decode_attention: workspace of %zu bytes, %zu needed", workspace_bytes,
                         need);
            KVHP_REQUIRE(aligned16(ws), KVHP_ERR_INVALID, "decode_attention: workspace not 16-byte aligned");
        }
        char* base = static_cast<char*>(ws);
        const size_t tk = align256(sizeof(uint32_t) * (size_t)batch * hkv);
        const size_t ob = align256(sizeof(float) * (size_t)batch * hq * plan.nsplit * d);
        a.tickets = reinterpret_cast<uint32_t*>(base);
        a.ws_o = reinterpret_cast<float*>(base + tk);
        a.ws_ml = reinterpret_cast<float*>(base + tk + ob);
    }
    dim3 grid(plan.nsplit, hkv, batch);
    const bool ok = d == 64 ? dispatch_g<64>(G, a, grid, paged, s)
                            : dispatch_g<128>(G, a, grid, paged, s);
    if (!ok) return fail(KVHP_ERR_UNSUPPORTED, "decode_attention: group size %d", G);
    return check_launch("decode_attention");
}

}  // namespace kvhp

using namespace kvhp;

extern "C" int kvhp_decode_auto_splits(int batch, int num_kv_heads, int head_dim,
                                       int max_seq_len) {
    (void)head_dim;
    return make_plan(batch, num_kv_heads, max_seq_len, 0).nsplit;
}

extern "C" size_t kvhp_decode_workspace_bytes(int batch, int num_q_heads,
                                              int num_kv_heads, int head_dim,
                                              int max_seq_len, int num_splits) {
    if (batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0) return 0;
    return workspace_bytes_for(batch, num_q_heads, num_kv_heads, head_dim,
                               make_plan(batch, num_kv_heads, max_seq_len, num_splits));
}

extern "C" int kvhp_decode_workspace_init(void* workspace, size_t workspace_bytes,
                                          void* stream) {
    clear_error();
    if (!workspace || workspace_bytes == 0) return KVHP_OK;
    KVHP_HIP(hipMemsetAsync(workspace, 0, workspace_bytes, static_cast<hipStream_t>(stream)),
             "hipMemsetAsync(workspace)");
    return KVHP_OK;
}

extern "C" int kvhp_decode_attention(const void* q, const kvhp_kv_view* k_view,
                                     const kvhp_kv_view* v_view, const int32_t* seq_lens,
                                     void* out, int batch, int num_q_heads,
                                     int num_kv_heads, int head_dim, int max_seq_len,
                                     int num_splits, void* workspace,
                                     size_t workspace_bytes, void* stream) {
    clear_error();
    KVHP_REQUIRE(seq_lens, KVHP_ERR_INVALID, "decode_attention: null seq_lens");
    return decode_attention_impl(q, k_view, v_view, seq_lens, 0, out, batch, num_q_heads,
                                 num_kv_heads, head_dim, max_seq_len, num_splits, workspace,
                                 workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int kvhp_decode_gqa(const void* q, const void* k_cache, const void* v_cache,
                               void* out, int total_seq_len, int num_q_heads,
                               int num_kv_heads, int max_seq, int head_dim, void* stream) {
    clear_error();
    if (total_seq_len <= 0) return KVHP_OK;  // decode_attention.cu:126
    KVHP_REQUIRE(k_cache && v_cache, KVHP_ERR_INVALID, "decode_gqa: null cache");
    KVHP_REQUIRE(total_seq_len <= max_seq, KVHP_ERR_INVALID,
                 "decode_gqa: total_seq_len %d > max_seq %d", total_seq_len, max_seq);
    hipStream_t s = static_cast<hipStream_t>(stream);
    kvhp_kv_view kv{};
    kv.data = k_cache;
    kv.stride_b = 0;
    kv.stride_h = (int64_t)max_seq * head_dim;
    kv.stride_s = head_dim;
    kv.stride_d = 1;
    kvhp_kv_view vv = kv;
    vv.data = v_cache;
    return decode_attention_impl(q, &kv, &vv, nullptr, total_seq_len, out, 1, num_q_heads,
                                 num_kv_heads, head_dim, total_seq_len, 0, nullptr, 0, s);
}
