// prefill.hip -- causal flash attention for prefill on CDNA4 fp16 MFMA (gfx950).
//
// Work decomposition: a 256-thread workgroup (4 waves) owns 64 query rows of
// one query head; each wave owns 16 rows.  The workgroup walks 64-key tiles
// from key 0 to the diagonal, staging each K and V tile once in LDS for its
// four waves.
//
// Per tile and wave, everything is computed transposed so that one lane owns
// one query row for the whole softmax (no cross-lane row bookkeeping beyond
// a 4-lane max/sum):
//   S^T = K Q^T   v_mfma_f32_16x16x32_f16, A = K rows from LDS (16 B reads),
//                 B = Q^T held in registers for the whole loop.
//                 Lane l gets scores of query row l%16 for keys 4(l/16)+e of
//                 each 16-key block.
//   softmax       fp32, log2 domain, causal mask on the diagonal tile only.
//   O^T += V^T P^T  A = V^T gathered from the LDS V tile, B = P^T converted
//                 to fp16 in registers straight from the S^T accumulators
//                 (key slot (g,e) of the k-step maps to key 4g+e of the first
//                 and 16+4g+e of the second 16-key block, in both operands).
// Output rows are normalised once at the end and stored as fp16.
//
// Scheduling: grid x enumerates query heads so that the G heads of one KV
// head map to the same XCD (x % 8), y enumerates query blocks longest-first.
// With a page pool, the workgroups of the first query head of each KV group
// also write the K/V rows of their own 64-key diagonal tile into the pages
// (every key row is written exactly once, from registers already loaded).
//
// Roofline: MFMA-bound for long prompts; algorithmic work 4*D*Hq*S(S+1)/2
// flops (two causal contractions).
#include "kvhp_internal.h"

#include <cmath>

namespace kvhp {

namespace {

constexpr int kBM = 64;     // query rows per workgroup
constexpr int kBN = 64;     // keys per tile
constexpr int kThreads = 256;

struct PrefillArgs {
    const f16* q;           // [B][S][Hq][D]
    const f16* k;           // [B][S][Hkv][D]
    const f16* v;
    f16* out;               // [B][S][Hq][D]
    f16* pool_k;            // optional page pool [Hkv][P][16][D]
    f16* pool_v;
    const int32_t* bt;      // [B][max_pages]
    int max_pages;
    int num_pages;
    int S, Hq, Hkv, G;
    int n_qblk;
    float scale_log2;
};

template <int D>
__global__ void __launch_bounds__(kThreads)
prefill_mfma_kernel(const PrefillArgs a) {
    constexpr int NC = D / 32;          // k-chunks of the QK contraction
    constexpr int ND = D / 16;          // 16-dim blocks of the output
    constexpr int CPR = D / 8;          // 16-byte chunks per row
    constexpr int LDR = D + 8;          // LDS row pitch in halfs (bank skew)
    constexpr int LOADS = kBN * CPR / kThreads;

    __shared__ f16 Ks[kBN * LDR];
    __shared__ f16 Vs[kBN * LDR];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int g = lane >> 4;
    const int col = lane & 15;

    const int kvh = blockIdx.x % a.Hkv;
    const int qh = kvh * a.G + blockIdx.x / a.Hkv;
    const int qblk = a.n_qblk - 1 - (int)blockIdx.y;
    const int b = blockIdx.z;
    const int q0 = qblk * kBM;
    const int S = a.S;
    const int64_t qrow_stride = (int64_t)a.Hq * D;
    const int64_t kvrow_stride = (int64_t)a.Hkv * D;
    const f16* qb = a.q + (int64_t)b * S * qrow_stride + (int64_t)qh * D;
    const f16* kb = a.k + (int64_t)b * S * kvrow_stride + (int64_t)kvh * D;
    const f16* vb = a.v + (int64_t)b * S * kvrow_stride + (int64_t)kvh * D;
    const bool write_pages = a.pool_k != nullptr && (qh % a.G) == 0;

    // This lane's query row, as the B operand (Q^T): dims 32c + 8g .. +8.
    const int my_row = q0 + wave * 16 + col;
    half8 qop[NC];
    if (my_row < S) {
#pragma unroll
        for (int c = 0; c < NC; ++c)
            qop[c] = load_half8(qb + (int64_t)my_row * qrow_stride + 32 * c + 8 * g);
    } else {
#pragma unroll
        for (int c = 0; c < NC; ++c) qop[c] = half8{};
    }

    floatx4 o[ND];
#pragma unroll
    for (int i = 0; i < ND; ++i) o[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -1e30f;
    float l_part = 0.f;

    const int last_row = min(q0 + kBM, S) - 1;
    const int n_tiles = last_row / kBN + 1;
    const int wave_last_row = q0 + wave * 16 + 15;

    for (int kt = 0; kt < n_tiles; ++kt) {
        const int k0 = kt * kBN;
        __syncthreads();
        // ---- stage K and V tiles (rows past S are zero).
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const int idx = i * kThreads + tid;
            const int r = idx / CPR;
            const int ch = idx % CPR;
            const int key = k0 + r;
            half8 kv = {}, vv = {};
            if (key < S) {
                kv = load_half8(kb + (int64_t)key * kvrow_stride + 8 * ch);
                vv = load_half8(vb + (int64_t)key * kvrow_stride + 8 * ch);
                if (write_pages && key >= q0 && key / kPage < a.max_pages) {
                    int pid = a.bt[(int64_t)b * a.max_pages + key / kPage];
                    if (pid >= 0 && pid < a.num_pages) {
                        const int64_t dst =
                            (((int64_t)kvh * a.num_pages + pid) * kPage + key % kPage) * D + 8 * ch;
                        store_half8(a.pool_k + dst, kv);
                        store_half8(a.pool_v + dst, vv);
                    }
                }
            }
            *reinterpret_cast<half8*>(&Ks[r * LDR + 8 * ch]) = kv;
            *reinterpret_cast<half8*>(&Vs[r * LDR + 8 * ch]) = vv;
        }
        __syncthreads();
        if (k0 > wave_last_row) continue;  // tile entirely above this wave's rows

        // ---- S^T = K Q^T: four 16-key blocks.
        floatx4 sc[4];
#pragma unroll
        for (int kb4 = 0; kb4 < 4; ++kb4) {
            sc[kb4] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const half8 kop =
                    *reinterpret_cast<const half8*>(&Ks[(16 * kb4 + col) * LDR + 32 * c + 8 * g]);
                sc[kb4] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop, qop[c], sc[kb4], 0, 0, 0);
            }
        }
        // ---- mask, running max for this lane's row (shared by 4 lanes).
        const bool diag = k0 + kBN - 1 > q0 + wave * 16;
        float tmax = -INFINITY;
#pragma unroll
        for (int kb4 = 0; kb4 < 4; ++kb4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int key = k0 + 16 * kb4 + 4 * g + e;
                float x = sc[kb4][e] * a.scale_log2;
                if (diag && (key > my_row || key >= S)) x = -INFINITY;
                sc[kb4][e] = x;
                tmax = fmaxf(tmax, x);
            }
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const float mn = fmaxf(m_run, tmax);
        const float alpha = fast_exp2(m_run - mn);
        m_run = mn;
        l_part *= alpha;
#pragma unroll
        for (int i = 0; i < ND; ++i) o[i] *= alpha;

        // ---- P^T operands (fp16) for the two 32-key k-steps.
        half8 pop[2];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float p0 = fast_exp2(sc[2 * ks][e] - mn);
                const float p1 = fast_exp2(sc[2 * ks + 1][e] - mn);
                l_part += p0 + p1;
                pop[ks][e] = static_cast<f16>(p0);
                pop[ks][4 + e] = static_cast<f16>(p1);
            }
        }
        // ---- O^T += V^T P^T.
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
            for (int db = 0; db < ND; ++db) {
                half8 vop;
                const int d = 16 * db + col;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    vop[e] = Vs[(32 * ks + 4 * g + e) * LDR + d];
                    vop[4 + e] = Vs[(32 * ks + 16 + 4 * g + e) * LDR + d];
                }
                o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop, pop[ks], o[db], 0, 0, 0);
            }
        }
    }

    float l_tot = l_part;
    l_tot += __shfl_xor(l_tot, 16);
    l_tot += __shfl_xor(l_tot, 32);
    if (my_row < S) {
        const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
        f16* orow = a.out + ((int64_t)b * S + my_row) * qrow_stride + (int64_t)qh * D;
#pragma unroll
        for (int db = 0; db < ND; ++db) {
            half4 h;
#pragma unroll
            for (int e = 0; e < 4; ++e) h[e] = static_cast<f16>(o[db][e] * inv);
            *reinterpret_cast<half4*>(orow + 16 * db + 4 * g) = h;
        }
    }
}

// Any head_dim <= 256 / any alignment: one wave per (query head, row),
// online softmax over keys 0..row.  Optionally writes the page pool too
// (from the first query head of each group, one wave per key row).
__global__ void __launch_bounds__(kWave)
prefill_generic_kernel(const PrefillArgs a, int D) {
    const int lane = threadIdx.x;
    const int qh = blockIdx.x;
    const int row = blockIdx.y;
    const int b = blockIdx.z;
    const int kvh = qh / a.G;
    const int S = a.S;
    const int64_t qrs = (int64_t)a.Hq * D, kvrs = (int64_t)a.Hkv * D;
    const f16* qp = a.q + ((int64_t)b * S + row) * qrs + (int64_t)qh * D;
    const f16* kb = a.k + (int64_t)b * S * kvrs + (int64_t)kvh * D;
    const f16* vb = a.v + (int64_t)b * S * kvrs + (int64_t)kvh * D;
    if (a.pool_k && qh % a.G == 0 && row / kPage < a.max_pages) {
        int pid = a.bt[(int64_t)b * a.max_pages + row / kPage];
        if (pid >= 0 && pid < a.num_pages) {
            const int64_t dst = (((int64_t)kvh * a.num_pages + pid) * kPage + row % kPage) * D;
            for (int d = lane; d < D; d += kWave) {
                a.pool_k[dst + d] = kb[(int64_t)row * kvrs + d];
                a.pool_v[dst + d] = vb[(int64_t)row * kvrs + d];
            }
        }
    }
    float qv[4], acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int d = lane + kWave * i;
        qv[i] = d < D ? static_cast<float>(qp[d]) : 0.f;
        acc[i] = 0.f;
    }
    float m = -1e30f, l = 0.f;
    for (int t = 0; t <= row; ++t) {
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = lane + kWave * i;
            if (d < D) dot = fmaf(qv[i], static_cast<float>(kb[(int64_t)t * kvrs + d]), dot);
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
            const float vv = d < D ? static_cast<float>(vb[(int64_t)t * kvrs + d]) : 0.f;
            acc[i] = fmaf(p, vv, acc[i] * al);
        }
        m = mn;
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    f16* op = a.out + ((int64_t)b * S + row) * qrs + (int64_t)qh * D;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int d = lane + kWave * i;
        if (d < D) op[d] = static_cast<f16>(acc[i] * inv);
    }
}

}  // namespace

int prefill_impl(const void* q, const void* k, const void* v, void* out, int64_t seq_len,
                 int hq, int hkv, int d, int batch, void* pool_k, void* pool_v,
                 const int32_t* bt, int max_pages, int num_pages, hipStream_t s) {
    if (seq_len <= 0 || batch <= 0) return KVHP_OK;
    KVHP_REQUIRE(q && k && v && out, KVHP_ERR_INVALID, "flash_prefill: null pointer");
    KVHP_REQUIRE(hq > 0 && hkv > 0 && hq % hkv == 0, KVHP_ERR_INVALID,
                 "flash_prefill: num_q_heads=%d must be a positive multiple of num_kv_heads=%d",
                 hq, hkv);
    KVHP_REQUIRE(d > 0 && d <= 256, KVHP_ERR_UNSUPPORTED,
                 "flash_prefill: head_dim=%d outside 1..256", d);
    KVHP_REQUIRE(seq_len <= (int64_t)1 << 30, KVHP_ERR_UNSUPPORTED,
                 "flash_prefill: seq_len %lld too large", (long long)seq_len);
    if (pool_k || pool_v || bt) {
        KVHP_REQUIRE(pool_k && pool_v && bt && max_pages > 0 && num_pages > 0,
                     KVHP_ERR_INVALID, "flash_prefill_paged: incomplete page pool arguments");
        KVHP_REQUIRE((int64_t)max_pages * kPage >= seq_len, KVHP_ERR_INVALID,
                     "flash_prefill_paged: %d pages per sequence cannot hold %lld tokens",
                     max_pages, (long long)seq_len);
    }
    PrefillArgs a;
    a.q = static_cast<const f16*>(q);
    a.k = static_cast<const f16*>(k);
    a.v = static_cast<const f16*>(v);
    a.out = static_cast<f16*>(out);
    a.pool_k = static_cast<f16*>(pool_k);
    a.pool_v = static_cast<f16*>(pool_v);
    a.bt = bt;
    a.max_pages = max_pages;
    a.num_pages = num_pages;
    a.S = static_cast<int>(seq_len);
    a.Hq = hq;
    a.Hkv = hkv;
    a.G = hq / hkv;
    a.scale_log2 = 1.4426950408889634f / std::sqrt(static_cast<float>(d));
    a.n_qblk = static_cast<int>((seq_len + kBM - 1) / kBM);

    const bool fast = (d == 64 || d == 128) && aligned16(q) && aligned16(k) && aligned16(v) &&
                      aligned16(out) && (!pool_k || (aligned16(pool_k) && aligned16(pool_v)));
    if (fast) {
        dim3 grid(hq, a.n_qblk, batch);
        if (d == 64)
            hipLaunchKernelGGL(prefill_mfma_kernel<64>, grid, dim3(kThreads), 0, s, a);
        else
            hipLaunchKernelGGL(prefill_mfma_kernel<128>, grid, dim3(kThreads), 0, s, a);
        return check_launch("flash_prefill");
    }
    dim3 grid(hq, static_cast<unsigned>(seq_len), batch);
    hipLaunchKernelGGL(prefill_generic_kernel, grid, dim3(kWave), 0, s, a, d);
    return check_launch("flash_prefill(generic)");
}

}  // namespace kvhp

using namespace kvhp;

extern "C" int kvhp_flash_prefill(const void* q, const void* k, const void* v, void* out,
                                  int64_t seq_len, int num_q_heads, int num_kv_heads,
                                  int head_dim, int batch, void* stream) {
    clear_error();
    return prefill_impl(q, k, v, out, seq_len, num_q_heads, num_kv_heads, head_dim, batch,
                        nullptr, nullptr, nullptr, 0, 0, static_cast<hipStream_t>(stream));
}

extern "C" int kvhp_flash_prefill_paged(const void* q, const void* k, const void* v,
                                        void* out, int64_t seq_len, int num_q_heads,
                                        int num_kv_heads, int head_dim, int batch,
                                        void* pool_k, void* pool_v,
                                        const int32_t* block_tables, int max_pages,
                                        int num_pages, void* stream) {
    clear_error();
    KVHP_REQUIRE(pool_k && pool_v && block_tables, KVHP_ERR_INVALID,
                 "flash_prefill_paged: null page pool / block table");
    return prefill_impl(q, k, v, out, seq_len, num_q_heads, num_kv_heads, head_dim, batch,
                        pool_k, pool_v, block_tables, max_pages, num_pages,
                        static_cast<hipStream_t>(stream));
}

extern "C" int kvhp_causal_gqa(const void* q, const void* k, const void* v, void* out,
                               int64_t seq_len, int64_t num_q_heads, int64_t num_kv_heads,
                               int64_t head_dim, void* stream) {
    clear_error();
    if (seq_len <= 0) return KVHP_OK;  // causal_attention.cu:133
    KVHP_REQUIRE(num_q_heads > 0 && num_q_heads < (1 << 20) && num_kv_heads > 0 &&
                     num_kv_heads < (1 << 20) && head_dim > 0 && head_dim < (1 << 20),
                 KVHP_ERR_INVALID, "causal_gqa: bad shape");
    return prefill_impl(q, k, v, out, seq_len, static_cast<int>(num_q_heads),
                        static_cast<int>(num_kv_heads), static_cast<int>(head_dim), 1, nullptr,
                        nullptr, nullptr, 0, 0, static_cast<hipStream_t>(stream));
}
