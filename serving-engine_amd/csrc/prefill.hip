// prefill.hip -- causal flash attention for prefill on CDNA4 fp16 MFMA (gfx950).
//
// Work decomposition: a 512-thread workgroup (8 waves) owns one KV head and
// a query block of 16*RB rows for all G query heads of that KV head -- G*RB
// = 8 units of (head, 16 rows), one unit per wave (RB = 8/G).  Each 64-key
// K/V tile is read from HBM once per workgroup and consumed by all 8 waves,
// so GQA heads share their K/V traffic.  Query blocks i and N-1-i are
// processed by the same workgroup, giving every workgroup the same causal
// work; grid x enumerates (pair, kv_head) with the kv head fastest.
//
// K/V staging: a 4-stage LDS ring (4 x 32 KB for D=128), filled by
// global_load_lds_dwordx4 (direct HBM->LDS, no VGPR round trip).  Tile t+3 is
// issued while tile t is consumed; before reading a stage each wave waits for
// its own loads of that stage (explicit s_waitcnt vmcnt(N)) and the
// workgroup meets at one barrier per tile.  Rows are stored with an XOR
// swizzle of their 16-byte chunks so that both the K reads (ds_read_b128)
// and the transposing V reads (ds_read_b64_tr_b16) are bank-conflict free.
//
// Per tile and unit, the contraction runs transposed so that one lane owns one
// query row for the whole online softmax:
//   S^T = K Q^T     v_mfma_f32_16x16x32_f16, A = K rows from LDS, B = Q^T
//                   held in registers.  Lane l gets keys 4(l/16)+e of each
//                   16-key block for query row l%16.
//   softmax         fp32 in the log2 domain; the causal mask is applied only on
//                   tiles that cross the diagonal; the running max is taken on
//                   raw scores and the rescale of O is skipped when no row's
//                   max moved.
//   O^T += V^T P^T  A = V^T read with ds_read_b64_tr_b16 (transposing 8-byte
//                   LDS reads), B = P^T converted to fp16 straight from the S^T
//                   accumulators: k-slot (g,e') of a 32-key step is key
//                   4g+e' (e'<4) or 16+4g+e'-4 in both operands.
//
// With a page pool, each workgroup also writes the K/V rows of its own query
// block into the pages after its outputs (every key row is written exactly
// once, bit-exact).
//
// Roofline: MFMA-bound for long prompts; algorithmic work 4*D*Hq*S(S+1)/2
// flops (the two causal contractions).
#include "kvhp_internal.h"

#include <cmath>

namespace kvhp {

namespace {

constexpr int kBN = 64;     // keys per tile

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
    int RB;                 // 16-row blocks per query block (fast kernel)
    int n_qblk;
    float scale_log2;
};

typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4v;
typedef __attribute__((address_space(3))) f16 lds_f16;
typedef __attribute__((address_space(3))) void lds_void;

// ds_read_b64_tr_b16: within each 16-lane block, lane i receives element
// (i % 4) of the 8-byte groups addressed by lanes 4k + i/4, k = 0..3.
__device__ __forceinline__ short4v lds_read_tr16(const f16* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)(lds_f16*)p);
}

__device__ __forceinline__ half8 cat_half8(short4v lo, short4v hi) {
    return __builtin_bit_cast(half8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// global_load_lds_dwordx4: lane l's 16 bytes land at lds_base + 16*l (M0
// holds the wave-uniform LDS base).  Issued as inline asm so that only the
// explicit vmcnt waits of the ring order it against the LDS reads: the
// compiler's own tracking cannot tell ring stages apart and would otherwise
// drain every in-flight stage before each read.
__device__ __forceinline__ void dma16(const f16* src, f16* lds_base) {
    const uint32_t m0v = static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((lds_void*)(lds_f16*)lds_base));
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 :: "s"(m0v), "v"(src) : "memory", "m0");
}

// s_waitcnt vmcnt(N) (expcnt / lgkmcnt left free).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Orders this wave's LDS accesses across the barrier without the vmcnt(0)
// drain a __syncthreads() fence implies (which would empty the DMA ring).
__device__ __forceinline__ void ring_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// A workgroup serves one KV head and a query block of 16*RB rows for all G
// query heads of that KV head: G*RB "units" of (head, 16 rows), at most 8,
// two per wave.  K/V tiles of 64 keys stream through a 4-stage LDS ring
// filled by direct global->LDS loads; rows are stored XOR-swizzled (16-byte
// chunk c of row r at position c ^ swz(r)) so the MFMA operand reads hit
// distinct banks without padding.  Query blocks i and N-1-i run in the same
// workgroup so every workgroup does the same causal work.
template <int D, int WAVES>
__global__ void __launch_bounds__(WAVES * kWave)
prefill_mfma_kernel(const PrefillArgs a) {
    constexpr int NTH = WAVES * kWave;  // threads per workgroup
    constexpr int NB = 8 / WAVES;       // units per wave (8 units per workgroup)
    constexpr int NC = D / 32;          // k-chunks of the QK contraction
    constexpr int ND = D / 16;          // 16-dim blocks of the output
    constexpr int CPR = D / 8;          // 16-byte chunks per row
    constexpr int RPI = kWave / CPR;    // rows per DMA instruction
    constexpr int IPW = kBN / RPI / WAVES;  // DMA instructions per wave per matrix
    constexpr int LPT = 2 * IPW;        // DMA loads per wave per tile (K + V)
    constexpr int TB = kBN * D;         // halfs per tile matrix
    constexpr int KSW = CPR - 1;        // K swizzle: c ^ (r & KSW)
    constexpr int VSW = CPR / 2 - 1;    // V swizzle: c ^ ((r & VSW) << 1)

    __shared__ __attribute__((aligned(16))) f16 st0[2 * TB];
    __shared__ __attribute__((aligned(16))) f16 st1[2 * TB];
    __shared__ __attribute__((aligned(16))) f16 st2[2 * TB];
    __shared__ __attribute__((aligned(16))) f16 st3[2 * TB];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS bases in SGPRs
    const int lane = tid & 63;
    const int g = lane >> 4;
    const int col = lane & 15;

    const int kvh = blockIdx.x % a.Hkv;
    const int pair = blockIdx.x / a.Hkv;
    const int b = blockIdx.y;
    const int S = a.S;
    const int G = a.G;
    const int RB = a.RB;
    const int BM = 16 * RB;
    const int nunits = G * RB;
    const int64_t qrs = (int64_t)a.Hq * D;     // q/out row stride
    const int64_t kvrs = (int64_t)a.Hkv * D;   // k/v row stride
    const f16* kb = a.k + (int64_t)b * S * kvrs + (int64_t)kvh * D;
    const f16* vb = a.v + (int64_t)b * S * kvrs + (int64_t)kvh * D;

    // DMA of tile tt into a stage: this wave's rows (wave*IPW + p)*RPI + lane/CPR.
    // Tiles past the last one re-load the last tile (an L2 hit): every path
    // issues the same loads, so the vmcnt bookkeeping stays exact.
    int last_tile = 0;
    auto issue = [&](f16* stg, int tt) {
        tt = min(tt, last_tile);
#pragma unroll
        for (int p = 0; p < IPW; ++p) {
            const int blk = wave * IPW + p;
            const int row = blk * RPI + lane / CPR;
            const int key = min(tt * kBN + row, S - 1);
            const int ck = (lane % CPR) ^ (row & KSW);
            const int cv = (lane % CPR) ^ ((row & VSW) << 1);
            dma16(kb + (int64_t)key * kvrs + 8 * ck, stg + blk * RPI * D);
            dma16(vb + (int64_t)key * kvrs + 8 * cv, stg + TB + blk * RPI * D);
        }
    };

    for (int pass = 0; pass < 2; ++pass) {
        const int qblk = pass == 0 ? pair : a.n_qblk - 1 - pair;
        if (pass == 1 && qblk <= pair) break;   // odd count: middle block once
        const int q0 = qblk * BM;

        // ---- this wave's units: u = wave + WAVES*i -> head kvh*G + u%G, rows r0..r0+15
        int r0[NB], qh[NB];
        bool uvalid[NB];
        half8 qop[NB][NC];
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int u = wave + WAVES * i;
            uvalid[i] = u < nunits;
            qh[i] = kvh * G + (uvalid[i] ? u % G : 0);
            r0[i] = q0 + 16 * (uvalid[i] ? u / G : 0);
            const int row = r0[i] + col;
            const bool live = uvalid[i] && row < S;
#pragma unroll
            for (int c = 0; c < NC; ++c)
                qop[i][c] = live ? load_half8(a.q + ((int64_t)b * S + row) * qrs +
                                              (int64_t)qh[i] * D + 32 * c + 8 * g)
                                 : half8{};
        }
        floatx4 o[NB][ND];
        float m_run[NB], l_part[NB];
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            m_run[i] = -1e30f;
            l_part[i] = 0.f;
#pragma unroll
            for (int db = 0; db < ND; ++db) o[i][db] = floatx4{0.f, 0.f, 0.f, 0.f};
        }

        const int last_row = min(q0 + BM, S) - 1;
        const int n_tiles = last_row / kBN + 1;
        last_tile = n_tiles - 1;

        wait_vmcnt<0>();  // q in registers before the ring: no compiler waits inside it
        ring_barrier();   // everyone is done with the previous pass's stages
        issue(st0, 0);
        issue(st1, 1);
        issue(st2, 2);

        // One tile on stage STG: wait for this wave's DMA of the tile (the two
        // later tiles stay in flight), barrier (all waves' DMA landed, the
        // previous stage is free), refill the previous stage with tile kt+3,
        // compute.
        auto step = [&](f16* stg, f16* next_stg, int kt) {
            wait_vmcnt<2 * LPT>();
            ring_barrier();
            issue(next_stg, kt + 3);

            const int k0 = kt * kBN;
            const f16* Kt = stg;
            const f16* Vt = stg + TB;

            // ---- S^T = K Q^T for both units, K operand shared.
            bool act[NB];
#pragma unroll
            for (int i = 0; i < NB; ++i) act[i] = uvalid[i] && k0 <= r0[i] + 15;
            floatx4 sc[NB][4];
#pragma unroll
            for (int i = 0; i < NB; ++i)
#pragma unroll
                for (int kb4 = 0; kb4 < 4; ++kb4) sc[i][kb4] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb4 = 0; kb4 < 4; ++kb4) {
                const int r = 16 * kb4 + col;
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    const int pos = (4 * c + g) ^ (r & KSW);
                    const half8 kop = *reinterpret_cast<const half8*>(&Kt[r * D + 8 * pos]);
#pragma unroll
                    for (int i = 0; i < NB; ++i)
                        sc[i][kb4] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop, qop[i][c],
                                                                            sc[i][kb4], 0, 0, 0);
                }
            }

            // ---- online softmax per unit; P^T operands straight from S^T.
            // Inactive units (invalid, or entirely above the diagonal) see
            // only -inf scores: alpha = 1 and p = 0 leave their state as is,
            // so every MFMA above and below runs unconditionally (no
            // branches, no conservative waits inside the ring).  The running
            // max is kept on raw scores (scale > 0), and the scale is folded
            // into the exp2 argument: p = 2^(s*c - m*c).
            half8 pop[NB][2];
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const int row = r0[i] + col;
                const bool diag = !act[i] || k0 + kBN - 1 > r0[i];
                if (diag) {
#pragma unroll
                    for (int kb4 = 0; kb4 < 4; ++kb4) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int key = k0 + 16 * kb4 + 4 * g + e;
                            if (!act[i] || key > row || key >= S) sc[i][kb4][e] = -INFINITY;
                        }
                    }
                }
                float tmax = -INFINITY;
#pragma unroll
                for (int kb4 = 0; kb4 < 4; ++kb4)
#pragma unroll
                    for (int e = 0; e < 4; ++e) tmax = fmaxf(tmax, sc[i][kb4][e]);
                tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
                tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
                const float mn = fmaxf(m_run[i], tmax);
                const float nmc = -mn * a.scale_log2;
                float ls = 0.f;
#pragma unroll
                for (int kb4 = 0; kb4 < 4; ++kb4) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float p = fast_exp2(fmaf(sc[i][kb4][e], a.scale_log2, nmc));
                        pop[i][kb4 / 2][(kb4 % 2) * 4 + e] = static_cast<f16>(p);
                        ls += p;
                    }
                }
                // Rescale only when some row's max moved (rare after the first
                // tiles): a wave-uniform branch.
                if (__builtin_amdgcn_read_exec() & __ballot(mn != m_run[i])) {
                    const float alpha = fast_exp2((m_run[i] - mn) * a.scale_log2);
                    l_part[i] *= alpha;
#pragma unroll
                    for (int db = 0; db < ND; ++db) o[i][db] *= alpha;
                }
                m_run[i] = mn;
                l_part[i] += ls;
            }

            // ---- O^T += V^T P^T; k-slot (g,e') of step ks is key
            //      ks*32 + (e' < 4 ? 4g + e' : 16 + 4g + e' - 4).
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const int R1 = 32 * ks + 4 * g + col / 4;
                const int R2 = R1 + 16;
                const int h = 4 * ((col % 4) & 1);
#pragma unroll
                for (int db = 0; db < ND; ++db) {
                    const int c = 2 * db + ((col % 4) >> 1);
                    const f16* p1 = &Vt[R1 * D + 8 * (c ^ ((R1 & VSW) << 1)) + h];
                    const f16* p2 = &Vt[R2 * D + 8 * (c ^ ((R2 & VSW) << 1)) + h];
                    const half8 vop = cat_half8(lds_read_tr16(p1), lds_read_tr16(p2));
#pragma unroll
                    for (int i = 0; i < NB; ++i)
                        o[i][db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop, pop[i][ks],
                                                                          o[i][db], 0, 0, 0);
                }
            }
        };

        for (int kt = 0; kt < n_tiles; kt += 4) {
            step(st0, st3, kt);
            if (kt + 1 < n_tiles) step(st1, st0, kt + 1);
            if (kt + 2 < n_tiles) step(st2, st1, kt + 2);
            if (kt + 3 < n_tiles) step(st3, st2, kt + 3);
        }
        wait_vmcnt<0>();  // drain the ring's trailing re-loads

        // ---- normalise and store: lane holds row r0+col, dims 16db + 4g + e.
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            float lt = l_part[i];
            lt += __shfl_xor(lt, 16);
            lt += __shfl_xor(lt, 32);
            const int row = r0[i] + col;
            if (!uvalid[i] || row >= S) continue;
            const float inv = lt > 0.f ? 1.f / lt : 0.f;
            f16* orow = a.out + ((int64_t)b * S + row) * qrs + (int64_t)qh[i] * D;
#pragma unroll
            for (int db = 0; db < ND; ++db) {
                half4 hv;
#pragma unroll
                for (int e = 0; e < 4; ++e) hv[e] = static_cast<f16>(o[i][db][e] * inv);
                *reinterpret_cast<half4*>(orow + 16 * db + 4 * g) = hv;
            }
        }

        // ---- pages: this query block's own K/V rows, once per KV head.
        if (a.pool_k) {
            for (int idx = tid; idx < BM * CPR; idx += NTH) {
                const int key = q0 + idx / CPR;
                const int ch = idx % CPR;
                if (key >= S || key / kPage >= a.max_pages) continue;
                const int pid = a.bt[(int64_t)b * a.max_pages + key / kPage];
                if (pid < 0 || pid >= a.num_pages) continue;
                const int64_t dst =
                    (((int64_t)kvh * a.num_pages + pid) * kPage + key % kPage) * D + 8 * ch;
                store_half8(a.pool_k + dst, load_half8(kb + (int64_t)key * kvrs + 8 * ch));
                store_half8(a.pool_v + dst, load_half8(vb + (int64_t)key * kvrs + 8 * ch));
            }
        }
        wait_vmcnt<0>();   // page stores complete before the next ring starts
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
    a.RB = 1;
    a.n_qblk = 0;

    const bool fast = (d == 64 || d == 128) && a.G <= 8 && aligned16(q) && aligned16(k) &&
                      aligned16(v) && aligned16(out) &&
                      (!pool_k || (aligned16(pool_k) && aligned16(pool_v)));
    if (fast) {
        // units of (head, 16 rows) per workgroup: G*RB <= 8, two per wave
        a.RB = 8 / a.G;
        const int bm = 16 * a.RB;
        a.n_qblk = static_cast<int>((seq_len + bm - 1) / bm);
        dim3 grid(hkv * ((a.n_qblk + 1) / 2), batch);
        constexpr int W = 8;  // waves per workgroup: one 16-row unit each
        if (d == 64)
            hipLaunchKernelGGL((prefill_mfma_kernel<64, W>), grid, dim3(W * kWave), 0, s, a);
        else
            hipLaunchKernelGGL((prefill_mfma_kernel<128, W>), grid, dim3(W * kWave), 0, s, a);
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
