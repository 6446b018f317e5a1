// decode.hip -- split-K decode attention over a GQA fp16 KV cache (gfx950).
//
// Work decomposition: one workgroup per (split, kv_head, sequence).  A split
// is a page-aligned chunk of `chunk` tokens (a multiple of 64; at most 64
// pages with a block table); the workgroup serves all G = Hq/Hkv query heads
// of its KV head, so every K/V byte is read from HBM exactly once (the
// reference re-reads each KV row once per query head,
// src/cuda/decode_attention_split.cu:40-49).  Balanced batches (below) run
// one wave per split.  Fixed chunks at D = 64, and single splits, run four
// waves per split that take its 32-token steps round robin and fold their
// (m, l, O) together in LDS: each wave's chain of dependent steps (~0.55 us
// each with one wave per CU) is a quarter as long.
//
// Per 32-token step (2 pages of 16 tokens), both contractions run on
// v_mfma_f32_16x16x32_f16 in transposed form, so that lane (g, col) owns
// query head `col` for the whole online softmax:
//   S^T = K Q^T     A = K rows from the LDS tile (lane: token col of a
//                   page, 16 B at dims 32c + 8g), B = Q^T held in
//                   registers (zero columns for heads >= G).
//   softmax         fp32 in the log2 domain; per-lane max over its 8 tokens,
//                   then v_permlane16/32_swap across the four lane rows (no
//                   LDS round trip); the rescale factor never leaves the lane
//                   and O is rescaled only when some head's max moved.
//   O^T += V^T P^T  A = V^T read from a padded LDS tile with
//                   ds_read_b64_tr_b16 (transposing 8-byte reads), B = P^T in
//                   fp16 straight from the S^T accumulators.
// K is fetched two steps ahead into registers and V one step ahead, both as
// whole rows per load (contiguous bytes; loading K straight in the MFMA
// layout, 64 bytes of each of 16 rows per load, cost ~5 % of HBM
// throughput), then staged through LDS: K back in the A layout, V for the
// transposed reads.  Non-temporal loads (the cache is streamed once) and
// identical loads on every path so the compiler keeps exact vmcnt waits.
// Up to 252 VGPRs and 17.9 KB LDS per wave at D=128: two waves per SIMD,
// eight per CU.
//
// Splits: a sequence whose keys fit one split gets its output written
// directly; otherwise each split stores (m, l, o[D]) in fp32 and a second,
// small launch combines them by log-sum-exp: decode_merge_kernel per (kv
// head, sequence), or decode_merge_rows_kernel per (query head, sequence)
// for fixed chunks with 64 KB or more of partials per kv head.
// An explicit split count cuts every sequence into chunks of one size (grid
// = split x kv head x sequence).  The automatic count for a batch of 8 or
// more balances on the device: every workgroup sums the batch's lengths,
// derives each sequence's chunk so that the batch has about one split per
// resident wave slot, and finds its own (sequence, split) by a wave scan of
// the per-sequence split counts (grid = kv head x split list), so a ragged
// batch fills the GPU once instead of leaving a partial second round.
//
// Roofline: HBM-bound; algorithmic bytes per (token, kv_head) are 4*D
// (K + V fp16) plus the q read and output write per query head.
#include "kvhp_internal.h"

#include <cmath>
#include <algorithm>
#include <mutex>
#include <type_traits>
#include <vector>

namespace kvhp {

namespace {

constexpr int kMaxSplits = 512;   // partials per (sequence, kv head)
constexpr int kMaxPagedChunk = 1024;  // tokens per split with a block table: one
                                      // page id per lane of a wave (64 pages)

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
    int Hq, Hkv;
    int chunk;             // tokens per split, multiple of 64 (fixed mode)
    int nsplit;            // split slots in the workspace
    int batch;             // sequences
    int balance;           // > 0: per-sequence chunks, about this many splits per kv head
                           // over the batch; 0: every sequence uses `chunk`
    int min_chunk;         // balanced: fewest tokens per split ...
    int max_chunk;         // ... and most (nsplit * max_chunk >= cap)
    int cap;               // tokens addressable per sequence
    int fixed_len;         // length of every sequence when seq_lens == nullptr
    float scale_log2;      // log2(e) / sqrt(D)
    // > 0: out is row-tiled ([B][Hq*D] in act_tiled_index order, this many
    // batch tiles; the batched model runner's o-projection input), written by
    // the kernels instantiated for it; 0: row-major.  (In the padding before
    // k_new: no other argument moves.)
    int out_tiles;
    // Fused append (k_new == nullptr: none): row b of k_new / v_new
    // [B][Hkv][D] is the token at position new_pos[b]; the split that covers
    // it writes it into its page (or its row of a strided view) before
    // reading it.
    const f16* k_new;
    const f16* v_new;
    const int32_t* new_pos;
    f16* pool_k;           // the K / V pools of the views, writable
    f16* pool_v;
};

__device__ __forceinline__ int seq_len_of(const DecodeArgs& a, int b) {
    return a.seq_lens ? a.seq_lens[b] : a.fixed_len;
}

// Keys of the whole batch (each length clamped to [0, cap]), summed by one
// full wave; every wave that calls it gets the same value.
__device__ __forceinline__ long long batch_keys(const DecodeArgs& a, int lane) {
    long long t = 0;
    for (int i = lane; i < a.batch; i += kWave) t += min(max(seq_len_of(a, i), 0), a.cap);
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) t += __shfl_xor(t, o);
    return t;
}

// Tokens per split of a sequence of L keys.  Fixed mode: the host's chunk.
// Balanced mode: the batch's keys are cut into about `balance` equal splits
// per kv head (so the grid fills the GPU's wave slots about once, whatever
// the spread of lengths), then each sequence's splits are evened out; the
// chunk is page-aligned, never above a.max_chunk, and ceil(L / chunk) <= nsplit.
// The split and merge kernels call this with the same arguments, so they
// agree on every sequence's split count.
__device__ __forceinline__ int chunk_of(const DecodeArgs& a, int L, long long keys) {
    if (a.balance <= 0 || L <= 0) return a.chunk;
    const int target = static_cast<int>(
        min(max((keys + a.balance - 1) / a.balance, (long long)a.min_chunk), (long long)a.max_chunk));
    const int n = min((L + target - 1) / target, a.nsplit);
    // ceil(L / n) <= target, or (n == nsplit) ceil(L / n) <= ceil(cap / nsplit):
    // both at most max_chunk, a multiple of the page, so the page-aligned
    // chunk stays within it, and ceil(L / chunk) <= n <= nsplit
    return ((L + n - 1) / n + kPage - 1) / kPage * kPage;
}

typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4v;
typedef __attribute__((address_space(3))) f16 lds_f16;

// ds_read_b64_tr_b16: within each 16-lane block, lane i receives element
// (i % 4) of the 8-byte groups addressed by lanes 4k + i/4, k = 0..3.
// So if lane j addresses the 4 consecutive elements [col0 + 4(j%4), +4) of
// row R(j/4), lane i gets column col0 + i of rows R(0..3): a 4 x 16 tile
// transposed into the MFMA operand layout.
__device__ __forceinline__ short4v lds_read_tr16(const f16* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)(lds_f16*)p);
}

__device__ __forceinline__ half8 cat_half8(short4v lo, short4v hi) {
    return __builtin_bit_cast(half8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// One workgroup of W waves per (split, kv_head, sequence); wave w takes the
// split's 32-token steps w, w+W, ... and the waves' states meet in LDS at
// the end (W = 1: the wave's state is the split's).  Both contractions
// are transposed so that lane (g, col) -- g = lane/16, col = lane%16 -- owns
// query head `col` of the KV head's group for the whole online softmax:
//   S^T = K Q^T   A = K rows of one 16-token page from k_lds (lane: token
//                 col, dims 32c+8g..+8), B = Q^T (lane:
//                 head col, same dims; zero for col >= G).  Lane (g, col)
//                 gets tokens 4g+e of the page for head col.
//   softmax       per head = per lane: in-lane max over its 8 tokens of the
//                 32-token step, then rows4_max; rescale factor lane-local.
//   O^T += V^T P^T  A = V^T from LDS by transposing 8-byte reads (dims
//                 16db+col, tokens 4g..4g+3 and 16+4g..16+4g+3), B = P^T in
//                 fp16 straight from the S^T accumulators (k-slot (g, e) is
//                 token 4g+e of page 0 for e < 4, of page 1 for e >= 4).
// K runs two of the wave's steps ahead in registers, V one; both are loaded as whole
// rows and staged through LDS (K for the A layout, V for the transposed
// reads).
template <int D, int G, bool PAGED, int W, bool TOUT = false>
__global__ void __launch_bounds__(W * kWave) __attribute__((amdgpu_waves_per_eu(2)))
decode_splitk_kernel(const DecodeArgs a) {
    static_assert(G >= 1 && G <= 16, "one MFMA column per query head");
    static_assert(W == 1 || W == 4, "one or four waves per split");
    constexpr int TOK = 32;          // tokens per step: 2 pages, one PV k-step
    constexpr int NC = D / 32;       // QK k-chunks
    constexpr int ND = D / 16;       // 16-dim output blocks
    constexpr int LPR = D / 8;       // lanes per V row (16 B each)
    constexpr int RPL = kWave / LPR; // V rows per wave load
    constexpr int NVL = TOK / RPL;   // V (and K) loads per step
    constexpr int VP = D + 16;       // V tile row pitch in halfs (bank skew)
    constexpr int KP = D + 8;        // K tile row pitch in halfs (bank skew)

    __shared__ __attribute__((aligned(16))) f16 v_lds_all[W][TOK * VP];
    __shared__ __attribute__((aligned(16))) f16 k_lds_all[W][TOK * KP];

    const int lane = threadIdx.x & (kWave - 1);
    // W waves split the split's 32-token steps round robin and meet in LDS.
    const int wv = W > 1 ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : 0;
    f16* const v_lds = v_lds_all[wv];
    f16* const k_lds = k_lds_all[wv];
    const int g = lane >> 4;
    const int col = lane & 15;
    int kvh, b, split, L, chunk;
    if (W == 1 && a.balance > 0) {
        // Balanced work list: blockIdx.y is the index of this split among
        // all splits of the batch in sequence order (sequences without keys
        // keep one, which writes their zero output), blockIdx.x the kv head,
        // so the grid's live workgroups come first and spread over every CU.
        // Every wave recomputes each sequence's split count and scans them,
        // 64 sequences a pass.
        kvh = blockIdx.x;
        const long long keys = batch_keys(a, lane);
        const int i = blockIdx.y;
        int base = 0;
        b = -1;
        split = 0;
        L = 0;
        chunk = a.chunk;
        for (int g0 = 0; g0 < a.batch; g0 += kWave) {
            const bool in = g0 + lane < a.batch;
            const int li = in ? min(max(seq_len_of(a, g0 + lane), 0), a.cap) : 0;
            const int ci = chunk_of(a, li, keys);
            const int ni = in ? (li > 0 ? (li + ci - 1) / ci : 1) : 0;
            int inc = ni;  // inclusive prefix over the lanes
#pragma unroll
            for (int o = 1; o < kWave; o <<= 1) {
                const int t = __shfl_up(inc, o);
                if (lane >= o) inc += t;
            }
            const int tot = __shfl(inc, kWave - 1);
            if (i < base + tot) {
                const int owner = __builtin_ctzll(__ballot(base + inc > i));
                b = g0 + owner;
                split = i - base - (__shfl(inc, owner) - __shfl(ni, owner));
                L = __shfl(li, owner);
                chunk = __shfl(ci, owner);
                break;
            }
            base += tot;
        }
        if (b < 0) return;   // past the batch's splits
        b = __builtin_amdgcn_readfirstlane(b);
        split = __builtin_amdgcn_readfirstlane(split);
        L = __builtin_amdgcn_readfirstlane(L);
        chunk = __builtin_amdgcn_readfirstlane(chunk);
    } else {
        split = blockIdx.x;
        kvh = blockIdx.y;
        b = blockIdx.z;
        L = seq_len_of(a, b);
        if (L > a.cap) L = a.cap;
        chunk = a.chunk;
    }
    const int64_t row0 = (int64_t)b * a.Hq + (int64_t)kvh * G;  // first q row
    const bool hvalid = col < G;
    const int nsb = L > 0 ? (L + chunk - 1) / chunk : 0;

    // Fused append: the split that covers the new position (the last split
    // if it lies beyond them) writes the row into its page (strided views:
    // its row) before its first K/V load and waits for the stores to
    // complete, so its own loads of that row return it -- the reference
    // appends before it attends (forward_gpu.cu:593-640), and only this
    // workgroup reads that row.  Invalid positions and page ids are dropped
    // as by kvhp_paged_append_kv; on a strided view positions at or past the
    // call's capacity, as kvhp_append_kv drops those past max_seq.
    int app_pos = -1;
    if (a.k_new) {
        const int p = a.new_pos[b];
        const int last = a.balance > 0 ? max(nsb, 1) - 1 : a.nsplit - 1;
        if (p >= 0 && split == min(p / chunk, last)) app_pos = p;
    }
    // Splits past the sequence's keys stop here (before any page-table
    // load), except the one that appends.
    if (split >= max(nsb, 1) && app_pos < 0) return;

    // Page ids of this split, one per lane (the host keeps a paged split to
    // at most 64 pages): one vector load here instead of a scalar load per
    // step on the critical path; steps fetch them with v_readlane.
    int pidv = 0;
    const int first_page = (split * chunk) >> 4;
    if constexpr (PAGED) {
        const int32_t* row = a.k.bt + (int64_t)b * a.k.max_pages;
        const int in_row = a.k.max_pages - first_page;
        if (in_row > 0) {
            int pid = row[first_page + (lane < in_row ? lane : in_row - 1)];
            pidv = pid < 0 ? 0 : (pid >= a.k.num_pages ? a.k.num_pages - 1 : pid);
        }
    }

    if constexpr (PAGED) {
        if (app_pos >= 0) {
            const int p = app_pos;
            constexpr int LPR0 = D / 8;
            const int pid = (p >> 4) < a.k.max_pages
                                ? a.k.bt[(int64_t)b * a.k.max_pages + (p >> 4)] : -1;
            if (pid >= 0 && pid < a.k.num_pages && lane < LPR0) {
                const int64_t src = ((int64_t)b * a.Hkv + kvh) * D + 8 * lane;
                const int64_t dst = kvh * a.k.stride_h +
                                    ((int64_t)pid * kPage + (p & 15)) * a.k.stride_s + 8 * lane;
                store_half8(a.pool_k + dst, load_half8(a.k_new + src));
                store_half8(a.pool_v + dst, load_half8(a.v_new + src));
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
    } else {
        if (app_pos >= 0) {
            const int p = app_pos;
            constexpr int LPR0 = D / 8;
            if (p < a.cap && lane < LPR0) {
                const int64_t src = ((int64_t)b * a.Hkv + kvh) * D + 8 * lane;
                const int64_t dk = b * a.k.stride_b + kvh * a.k.stride_h + p * a.k.stride_s + 8 * lane;
                const int64_t dv = b * a.v.stride_b + kvh * a.v.stride_h + p * a.v.stride_s + 8 * lane;
                store_half8(a.pool_k + dk, load_half8(a.k_new + src));
                store_half8(a.pool_v + dv, load_half8(a.v_new + src));
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
    }

    if (L <= 0) {
        if (split == 0) {
            const half8 z = {};
            for (int i = lane; i < G * LPR; i += kWave)
                if constexpr (TOUT)
                    store_half8(a.out + act_tiled_index(b, (int64_t)(kvh * G + i / LPR) * D +
                                                               8 * (i % LPR), a.out_tiles), z);
                else
                    store_half8(a.out + (row0 + i / LPR) * D + 8 * (i % LPR), z);
        }
        return;
    }
    if (split >= nsb) return;
    const int t_begin = split * chunk;
    const int t_end = min(L, t_begin + chunk);
    const int n_iter = (t_end - t_begin + TOK - 1) / TOK;
    const int last_tok = t_end - 1;
    const int last_pi = last_tok >> 4;
    const int last_slot = last_tok & 15;

    const int64_t ssk = a.k.stride_s, ssv = a.v.stride_s;
    const f16* kbase;
    const f16* vbase;
    if constexpr (PAGED) {  // K and V share one block table
        kbase = a.k.data + kvh * a.k.stride_h;
        vbase = a.v.data + kvh * a.v.stride_h;
    } else {
        kbase = a.k.data + b * a.k.stride_b + kvh * a.k.stride_h;
        vbase = a.v.data + b * a.v.stride_b + kvh * a.v.stride_h;
    }

    // B operand of S^T: lane (g, col) holds q[head col][dims 32c + 8g .. +8].
    half8 qb[NC];
    if (hvalid) {
        const f16* qp = a.q + (row0 + col) * D + 8 * g;
#pragma unroll
        for (int c = 0; c < NC; ++c) qb[c] = load_half8(qp + 32 * c);
    } else {
#pragma unroll
        for (int c = 0; c < NC; ++c) qb[c] = half8{};
    }

    const int vrow = lane / LPR;
    const int vdim = 8 * (lane % LPR);

    // Page t of the step starting at T0, clamped into the split: a
    // wave-uniform base pointer, plus the last row a lane may read in it
    // (rows past the split's last token re-read its last row, so every load
    // is in bounds and finite, and prefetches are unconditional).  Lane
    // offsets inside a page are 32-bit: one saddr + voffset load each.
    auto page_base = [&](const f16* base, int64_t ss, int T0, int t, int& lim) {
        const int pu = (T0 >> 4) + t;
        const int pi = min(pu, last_pi);
        lim = pu >= last_pi ? last_slot : kPage - 1;
        int64_t row;
        if constexpr (PAGED)
            row = (int64_t)__builtin_amdgcn_readlane(pidv, pi - first_page) * kPage;
        else
            row = (int64_t)pi * kPage;
        return reinterpret_cast<const char*>(base + row * ss);
    };

    half8 kbuf[2][NVL];    // [ring slot][load]: whole rows, as V
    half8 vbuf[NVL];
    // Row pitch in bytes.  view_fast_ok admits stride_s < 2^26 halfs, so a
    // row offset inside a page, at most 15 pitches, stays below 2^31: a full
    // 32-bit multiply (a 24-bit one would drop the pitch's high bits).
    const uint32_t kss = static_cast<uint32_t>(ssk) * 2u;
    const uint32_t vss = static_cast<uint32_t>(ssv) * 2u;

    // K and V are fetched the same way: lane (vrow, vdim) loads 16 bytes of
    // row RPL*j + vrow, so each load covers RPL whole rows (contiguous
    // bytes; the MFMA layout, 64 bytes of 16 rows per load, cost ~5 % of HBM
    // throughput).  K reaches its operand layout through k_lds.
    auto load_k = [&](auto S_, int T0) {
        constexpr int S = decltype(S_)::value;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            int lim;
            const char* pb = page_base(kbase, ssk, T0, t, lim);
#pragma unroll
            for (int j = t * (kPage / RPL); j < (t + 1) * (kPage / RPL); ++j) {
                const int s0 = ((RPL * j) & (kPage - 1)) + vrow;
                const uint32_t off = static_cast<uint32_t>(min(s0, lim)) * kss + 2u * vdim;
                kbuf[S][j] = load_half8_stream(reinterpret_cast<const f16*>(pb + off));
            }
        }
    };
    auto load_v = [&](int T0) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            int lim;
            const char* pb = page_base(vbase, ssv, T0, t, lim);
#pragma unroll
            for (int j = t * (kPage / RPL); j < (t + 1) * (kPage / RPL); ++j) {
                const int s0 = ((RPL * j) & (kPage - 1)) + vrow;
                const uint32_t off = static_cast<uint32_t>(min(s0, lim)) * vss + 2u * vdim;
                vbuf[j] = load_half8_stream(reinterpret_cast<const f16*>(pb + off));
            }
        }
    };

    float m_run = -1e30f;  // running max of raw scores for head col
    float l_part = 0.f;    // this lane's share of the softmax denominator
    floatx4 o[ND];         // O^T: lane (g, col) holds dims 16db + 4g + e of head col
#pragma unroll
    for (int db = 0; db < ND; ++db) o[db] = floatx4{0.f, 0.f, 0.f, 0.f};
    const float sc = a.scale_log2;
    const f16* vrd = &v_lds[(4 * g + col / 4) * VP + 4 * (col % 4)];

    auto step = [&](auto S_, auto PFK_, auto PFV_, int it) {
        constexpr int S = decltype(S_)::value;
        constexpr bool PFK = decltype(PFK_)::value;
        constexpr bool PFV = decltype(PFV_)::value;
        const int T0 = t_begin + TOK * it;

        // ---- S^T = K Q^T for the two pages of the step: K rows into LDS,
        //      back in the A layout (lane (g, col): token col, dims 32c+8g).
#pragma unroll
        for (int j = 0; j < NVL; ++j)
            *reinterpret_cast<half8*>(&k_lds[(RPL * j + vrow) * KP + vdim]) = kbuf[S][j];
        if constexpr (PFK) load_k(S_, T0 + 2 * W * TOK);
        floatx4 C[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            C[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const half8 ka = *reinterpret_cast<const half8*>(&k_lds[(16 * t + col) * KP + 32 * c + 8 * g]);
                C[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qb[c], C[t], 0, 0, 0);
            }
        }

        // ---- tokens past the split (only in its last step).
        if (T0 + TOK > t_end) {
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (T0 + 16 * t + 4 * g + e >= t_end) C[t][e] = -INFINITY;
        }

        // ---- running max of head col, rescale factor, P^T in fp16.
        float mx = fmaxf(fmaxf(fmaxf(C[0][0], C[0][1]), fmaxf(C[0][2], C[0][3])),
                         fmaxf(fmaxf(C[1][0], C[1][1]), fmaxf(C[1][2], C[1][3])));
        mx = rows4_max(mx);
        const float mn = fmaxf(m_run, mx);
        const float alpha = fast_exp2((m_run - mn) * sc);
        m_run = mn;
        const float nm = hvalid ? -mn * sc : -INFINITY;  // padding heads get p = 0
        half8 pt;
        float ps = 0.f;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const f16 ph = static_cast<f16>(fast_exp2(fmaf(C[t][e], sc, nm)));
                pt[4 * t + e] = ph;
                ps += static_cast<float>(ph);
            }
        l_part = fmaf(l_part, alpha, ps);

        // ---- V tile into LDS, then the next V tile into the registers.
#pragma unroll
        for (int j = 0; j < NVL; ++j)
            *reinterpret_cast<half8*>(&v_lds[(RPL * j + vrow) * VP + vdim]) = vbuf[j];
        if constexpr (PFV) load_v(T0 + W * TOK);

        // Rescale O only when some head's running max moved.
        if (__builtin_amdgcn_read_exec() & __ballot(alpha != 1.f)) {
#pragma unroll
            for (int db = 0; db < ND; ++db)
#pragma unroll
                for (int e = 0; e < 4; ++e) o[db][e] *= alpha;
        }

        // ---- O^T += V^T P^T.
#pragma unroll
        for (int db = 0; db < ND; ++db) {
            const half8 va = cat_half8(lds_read_tr16(vrd + 16 * db),
                                       lds_read_tr16(vrd + 16 * VP + 16 * db));
            o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pt, o[db], 0, 0, 0);
        }
    };

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using Pf = std::true_type;
    using NoPf = std::false_type;
    // This wave's steps: wv, wv + W, wv + 2W, ... (n_w of them).
    const int n_w = n_iter > wv ? (n_iter - wv + W - 1) / W : 0;
    if (n_w > 0) {
        const int s0 = t_begin + TOK * wv;
        load_k(I0{}, s0);
        load_v(s0);
        load_k(I1{}, s0 + W * TOK);
        int j = 0;
        for (; j + 3 < n_w; j += 2) {
            step(I0{}, Pf{}, Pf{}, wv + W * j);
            step(I1{}, Pf{}, Pf{}, wv + W * (j + 1));
        }
        // tail: at most three steps, no loads past the split
        if (j + 2 < n_w) {
            step(I0{}, Pf{}, Pf{}, wv + W * j);
            step(I1{}, NoPf{}, Pf{}, wv + W * (j + 1));
            step(I0{}, NoPf{}, NoPf{}, wv + W * (j + 2));
        } else if (j + 1 < n_w) {
            step(I0{}, NoPf{}, Pf{}, wv + W * j);
            step(I1{}, NoPf{}, NoPf{}, wv + W * (j + 1));
        } else {
            step(I0{}, NoPf{}, NoPf{}, wv + W * j);
        }
    }

    if constexpr (W > 1) {
        // ---- the W waves' (m, l, O) meet in LDS: waves 1.. write theirs
        //      into their own K tile (free now: 64 (D + 8) bytes, exactly
        //      D/4 + 2 floats per lane), wave 0 folds them in.
        float* xs = reinterpret_cast<float*>(k_lds);
        if (wv > 0) {
#pragma unroll
            for (int db = 0; db < ND; ++db)
                *reinterpret_cast<floatx4*>(&xs[(db * kWave + lane) * 4]) = o[db];
            xs[ND * kWave * 4 + 2 * lane] = m_run;
            xs[ND * kWave * 4 + 2 * lane + 1] = l_part;
        }
        __syncthreads();
        if (wv > 0) return;
#pragma unroll
        for (int w = 1; w < W; ++w) {
            const float* xw = reinterpret_cast<const float*>(k_lds_all[w]);
            const float mw = xw[ND * kWave * 4 + 2 * lane];
            const float lw = xw[ND * kWave * 4 + 2 * lane + 1];
            const float mn = fmaxf(m_run, mw);
            const float a0 = fast_exp2((m_run - mn) * sc);
            const float a1 = fast_exp2((mw - mn) * sc);
            l_part = l_part * a0 + lw * a1;
#pragma unroll
            for (int db = 0; db < ND; ++db)
                o[db] = o[db] * a0 + *reinterpret_cast<const floatx4*>(&xw[(db * kWave + lane) * 4]) * a1;
            m_run = mn;
        }
    }

    const float l_tot = rows4_sum(l_part);
    if (!hvalid) return;
    const int64_t qrow = row0 + col;
    if (nsb == 1) {
        const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
        f16* orow = a.out + qrow * D + 4 * g;
#pragma unroll
        for (int db = 0; db < ND; ++db) {
            half4 h;
#pragma unroll
            for (int e = 0; e < 4; ++e) h[e] = static_cast<f16>(o[db][e] * inv);
            if constexpr (TOUT)
                *reinterpret_cast<half4*>(
                    a.out + act_tiled_index(b, (int64_t)(kvh * G + col) * D + 4 * g + 16 * db,
                                            a.out_tiles)) = h;
            else
                *reinterpret_cast<half4*>(orow + 16 * db) = h;
        }
        return;
    }
    const int64_t prow = qrow * a.nsplit + split;
    float* po = a.ws_o + prow * D + 4 * g;
#pragma unroll
    for (int db = 0; db < ND; ++db) *reinterpret_cast<floatx4*>(po + 16 * db) = o[db];
    if (g == 0) {
        a.ws_ml[prow * 2] = m_run * sc;  // log2 units
        a.ws_ml[prow * 2 + 1] = l_tot;
    }
}

// Log-sum-exp merge of the split partials of one (kv_head, sequence), four
// waves per workgroup, one memory round trip: lane (head h, 8 dims) of wave w
// folds splits w, w+4, w+8, ... into a running (max M, sum S, weighted o)
// with the (m, l) and o loads of U splits in flight at once; the four wave
// states then meet in LDS.  Partials hold o unnormalised and its sum l
// relative to the split's own max m (log2 units).
constexpr int kMergeWaves = 4;

template <int D, int G, bool TOUT = false>
__global__ void __launch_bounds__(kMergeWaves * kWave)
decode_merge_kernel(const DecodeArgs a) {
    constexpr int LPR = D / 8;          // lanes per head row (8 dims each)
    constexpr int HPP = kWave / LPR;    // heads per pass of one wave
    constexpr int NP = (G + HPP - 1) / HPP;
    constexpr int U = 8;                // splits in flight per lane (32 per round)
    __shared__ __attribute__((aligned(16))) float red_o[kMergeWaves - 1][NP][kWave][8];
    __shared__ float red_ms[kMergeWaves - 1][NP][kWave][2];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kvh = blockIdx.x;
    const int b = blockIdx.y;
    const int64_t row0 = (int64_t)b * a.Hq + (int64_t)kvh * G;
    int L = seq_len_of(a, b);
    if (L > a.cap) L = a.cap;
    if (L <= 0) return;
    const int chunk = chunk_of(a, L, a.balance > 0 ? batch_keys(a, lane) : 0);
    const int nsb = (L + chunk - 1) / chunk;
    if (nsb <= 1) return;  // written directly by the split kernel

    float M[NP], Sm[NP];
    floatx4 acc[NP][2];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        M[p] = -3.0e38f;   // below every partial max; exp2 of the gap is 0
        Sm[p] = 0.f;
        acc[p][0] = floatx4{0.f, 0.f, 0.f, 0.f};
        acc[p][1] = floatx4{0.f, 0.f, 0.f, 0.f};
        const int h = min(p * HPP + lane / LPR, G - 1);
        const int64_t prow = (row0 + h) * a.nsplit;
        const float* po = a.ws_o + prow * D + 8 * (lane % LPR);
        const float* pml = a.ws_ml + prow * 2;
        for (int j0 = wave; j0 < nsb; j0 += kMergeWaves * U) {
            float2 ml[U];
            floatx4 x[U][2];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int j = min(j0 + kMergeWaves * u, nsb - 1);
                ml[u] = *reinterpret_cast<const float2*>(pml + 2 * j);
                x[u][0] = *reinterpret_cast<const floatx4*>(po + (int64_t)j * D);
                x[u][1] = *reinterpret_cast<const floatx4*>(po + (int64_t)j * D + 4);
            }
            __builtin_amdgcn_sched_barrier(0);  // all U splits' loads in flight first
#pragma unroll
            for (int u = 0; u < U; ++u) {
                // splits past the end (clamped re-loads) get weight 0
                const float mu = j0 + kMergeWaves * u < nsb ? ml[u].x : -3.0e38f;
                const float mn = fmaxf(M[p], mu);
                const float al = fast_exp2(M[p] - mn);
                const float be = fast_exp2(mu - mn);
                acc[p][0] = acc[p][0] * al + x[u][0] * be;
                acc[p][1] = acc[p][1] * al + x[u][1] * be;
                Sm[p] = fmaf(Sm[p], al, ml[u].y * be);
                M[p] = mn;
            }
        }
        if (wave > 0) {
            float* r = red_o[wave - 1][p][lane];
            *reinterpret_cast<floatx4*>(r) = acc[p][0];
            *reinterpret_cast<floatx4*>(r + 4) = acc[p][1];
            red_ms[wave - 1][p][lane][0] = M[p];
            red_ms[wave - 1][p][lane][1] = Sm[p];
        }
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const int h = p * HPP + lane / LPR;
#pragma unroll
        for (int w = 0; w < kMergeWaves - 1; ++w) {
            const float mw = red_ms[w][p][lane][0];
            const float mn = fmaxf(M[p], mw);
            const float al = fast_exp2(M[p] - mn);
            const float be = fast_exp2(mw - mn);
            const float* r = red_o[w][p][lane];
            acc[p][0] = acc[p][0] * al + *reinterpret_cast<const floatx4*>(r) * be;
            acc[p][1] = acc[p][1] * al + *reinterpret_cast<const floatx4*>(r + 4) * be;
            Sm[p] = fmaf(Sm[p], al, red_ms[w][p][lane][1] * be);
            M[p] = mn;
        }
        if (h >= G) continue;
        const float inv = Sm[p] > 0.f ? 1.f / Sm[p] : 0.f;
        half8 hv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            hv[e] = static_cast<f16>(acc[p][0][e] * inv);
            hv[4 + e] = static_cast<f16>(acc[p][1][e] * inv);
        }
        if constexpr (TOUT)
            store_half8(a.out + act_tiled_index(b, (int64_t)(kvh * G + h) * D + 8 * (lane % LPR),
                                                a.out_tiles), hv);
        else
            store_half8(a.out + (row0 + h) * D + 8 * (lane % LPR), hv);
    }
}

// Merge for fixed chunks, one workgroup per (query head, sequence), so a
// small batch spreads its partials over B*Hq CUs instead of B*Hkv (at B=1,
// D=128, 64 splits, one workgroup per KV head pulls 133 KB through one CU).
// Lane (r, c): c = lane % LPR owns dims 8c..8c+7, r = lane / LPR is one of
// R split subsets; wave w's subset r takes splits (w*R + r) + k*W*R.  Every
// slot of the plan is loaded together with the length (no dependent round
// trip); slots past the sequence's last split are dropped by selects (their
// contents may be stale).  The subsets fold by lane exchanges, the waves
// through LDS.
template <int D, bool TOUT = false>
__global__ void __launch_bounds__(kMergeWaves * kWave)
decode_merge_rows_kernel(const DecodeArgs a) {
    constexpr int LPR = D / 8;
    constexpr int R = kWave / LPR;
    constexpr int STRIDE = kMergeWaves * R;
    constexpr int U = 4;   // splits per lane per round
    __shared__ __attribute__((aligned(16))) float red[kMergeWaves - 1][LPR][12];

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane % LPR;
    const int r = lane / LPR;
    const int b = blockIdx.y;
    const int64_t row = (int64_t)b * a.Hq + blockIdx.x;
    const int Lraw = seq_len_of(a, b);
    const float* po = a.ws_o + row * a.nsplit * D + 8 * c;
    const float* pml = a.ws_ml + row * a.nsplit * 2;

    float M = -3.0e38f, Sm = 0.f;
    floatx4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    int nsb = 0;
    for (int k = 0; k * STRIDE * U < a.nsplit; ++k) {   // uniform over the workgroup
        const int j0 = k * STRIDE * U + wave * R + r;
        float2 ml[U];
        floatx4 x[U][2];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = min(j0 + STRIDE * u, a.nsplit - 1);
            ml[u] = *reinterpret_cast<const float2*>(pml + 2 * j);
            x[u][0] = *reinterpret_cast<const floatx4*>(po + (int64_t)j * D);
            x[u][1] = *reinterpret_cast<const floatx4*>(po + (int64_t)j * D + 4);
        }
        if (k == 0) {   // first round: the length arrives with the loads
            const int L = min(Lraw, a.cap);
            if (L <= 0) return;
            nsb = (L + a.chunk - 1) / a.chunk;
            if (nsb <= 1) return;   // written directly by the split kernel
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const bool ok = j0 + STRIDE * u < nsb;
            const float mu = ok ? ml[u].x : -3.0e38f;
            const float lu = ok ? ml[u].y : 0.f;
            const floatx4 z = {0.f, 0.f, 0.f, 0.f};
            const float mn = fmaxf(M, mu);
            const float al = fast_exp2(M - mn);
            const float be = fast_exp2(mu - mn);
            acc0 = acc0 * al + (ok ? x[u][0] : z) * be;
            acc1 = acc1 * al + (ok ? x[u][1] : z) * be;
            Sm = fmaf(Sm, al, lu * be);
            M = mn;
        }
    }
    // fold the R subsets of the wave (lanes c, c + LPR, ...)
#pragma unroll
    for (int o = LPR; o < kWave; o <<= 1) {
        const float mo = __shfl_xor(M, o);
        const float so = __shfl_xor(Sm, o);
        floatx4 x0, x1;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x0[e] = __shfl_xor(acc0[e], o);
            x1[e] = __shfl_xor(acc1[e], o);
        }
        const float mn = fmaxf(M, mo);
        const float al = fast_exp2(M - mn);
        const float be = fast_exp2(mo - mn);
        acc0 = acc0 * al + x0 * be;
        acc1 = acc1 * al + x1 * be;
        Sm = Sm * al + so * be;
        M = mn;
    }
    if (wave > 0 && r == 0) {
        float* p = red[wave - 1][c];
        *reinterpret_cast<floatx4*>(p) = acc0;
        *reinterpret_cast<floatx4*>(p + 4) = acc1;
        p[8] = M;
        p[9] = Sm;
    }
    __syncthreads();
    if (wave != 0 || r != 0) return;
#pragma unroll
    for (int w = 0; w < kMergeWaves - 1; ++w) {
        const float* p = red[w][c];
        const float mn = fmaxf(M, p[8]);
        const float al = fast_exp2(M - mn);
        const float be = fast_exp2(p[8] - mn);
        acc0 = acc0 * al + *reinterpret_cast<const floatx4*>(p) * be;
        acc1 = acc1 * al + *reinterpret_cast<const floatx4*>(p + 4) * be;
        Sm = Sm * al + p[9] * be;
        M = mn;
    }
    const float inv = Sm > 0.f ? 1.f / Sm : 0.f;
    half8 hv;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        hv[e] = static_cast<f16>(acc0[e] * inv);
        hv[4 + e] = static_cast<f16>(acc1[e] * inv);
    }
    if constexpr (TOUT)
        store_half8(a.out + act_tiled_index(b, (int64_t)blockIdx.x * D + 8 * c, a.out_tiles), hv);
    else
        store_half8(a.out + row * D + 8 * c, hv);
}

// Append of one token per sequence into strided views (the fused append's
// fallback outside the fast kernel's shapes): element (b, h, d) of k_new /
// v_new [B][Hkv][D] to row new_pos[b] of sequence b, head h; positions
// outside [0, cap) are dropped.
__global__ void __launch_bounds__(256)
append_rows_strided_kernel(const f16* k_new, const f16* v_new, const KVDev k, const KVDev v,
                           const int32_t* new_pos, int batch, int hkv, int D, int cap,
                           f16* dst_k, f16* dst_v) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)batch * hkv * D) return;
    const int d = static_cast<int>(i % D);
    const int h = static_cast<int>((i / D) % hkv);
    const int b = static_cast<int>(i / ((int64_t)D * hkv));
    const int p = new_pos[b];
    if (p < 0 || p >= cap) return;
    dst_k[b * k.stride_b + h * k.stride_h + p * k.stride_s + d * k.stride_d] = k_new[i];
    dst_v[b * v.stride_b + h * v.stride_h + p * v.stride_s + d * v.stride_d] = v_new[i];
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
    // the fallback honours a row-tiled output at run time
    auto o_at = [&](int d) -> f16* {
        return a.out_tiles ? a.out + act_tiled_index(b, (int64_t)qh * D + d, a.out_tiles)
                           : a.out + row * D + d;
    };
    if (L <= 0) {
        for (int d = lane; d < D; d += kWave) *o_at(d) = f16(0);
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
        if (d < D) *o_at(d) = static_cast<f16>(acc[i] * inv);
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
        // Measured on MI355X (B=1..32, L=512..64K, D=64/128): chunks of about
        // L/64 tokens but never below 64, and at most ~6144 workgroups in
        // the grid.  Longer chunks starve the long sequences of a ragged
        // batch; shorter ones make the merge and per-workgroup set-up cost
        // more than they hide.  (A floor of 128 instead: the config-5 step
        // at ctx 2K 1522 vs 1549 tok/s, config 2 at 4K 12.6 vs 12.4 us; the
        // balanced batches keep their own 128-key minimum.)
        const int64_t units = (int64_t)batch * num_kv_heads;
        int per_split = (max_seq_len + 63) / 64;
        if (per_split < 64) per_split = 64;
        per_split = (per_split + 63) / 64 * 64;
        s = (max_seq_len + per_split - 1) / per_split;
        const int64_t grid_cap = units >= 6144 ? 1 : 6144 / units;
        if (s > grid_cap) s = static_cast<int>(grid_cap);
        // Small batches up to 512 keys: one split (four waves of at most four
        // 32-key steps each) and no merge launch, which costs more (~3 us)
        // than the three steps it saves a wave (~0.55 us each).
        if (batch < 8 && max_seq_len <= 512) s = 1;
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

// Workspace = fp32 o[B*Hq][nsplit][D] followed by (m, l)[B*Hq][nsplit]:
// exactly nsplit*B*Hq*(D+2) floats, the split_buffer size the reference's
// callers allocate (forward_gpu.cu:100, test_attention.cpp:124).  Only the
// fast kernels (D = 64 or 128) split, so the (m, l) block stays 16-B aligned.
// A paged split covers at most kMaxPagedChunk tokens.
Plan plan_for(int batch, int num_kv_heads, int max_seq_len, int num_splits, bool paged) {
    Plan p = make_plan(batch, num_kv_heads, max_seq_len, num_splits);
    if (paged && p.chunk > kMaxPagedChunk) {
        p.chunk = kMaxPagedChunk;
        p.nsplit = (max_seq_len + kMaxPagedChunk - 1) / kMaxPagedChunk;
    }
    return p;
}

size_t workspace_bytes_for(int batch, int hq, int hkv, int d, const Plan& p) {
    (void)hkv;
    if (p.nsplit <= 1) return 0;
    return sizeof(float) * (size_t)batch * hq * p.nsplit * (d + 2);
}

// Static split-partial scratch of kvhp_decode_attention_noalloc: 16 MiB
// per device (config 3's auto plan needs 11.2 MB), held until the process
// ends.  Kernels get it through the address hipGetSymbolAddress returns for
// the current device (scratch_address), never through the host-side name.
constexpr size_t kScratchBytes = size_t(16) << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

std::mutex g_scratch_mutex;
std::vector<void*> g_scratch;   // device address of `scratch`, per device

int scratch_address(void** out, hipStream_t s) {
    int dev = 0;
    KVHP_HIP(hipGetDevice(&dev), "hipGetDevice");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if ((int)g_scratch.size() <= dev) g_scratch.resize(dev + 1, nullptr);
    if (!g_scratch[dev]) {
        // The address is resolved once per device, outside any graph capture
        // (the symbol lookup is not a stream operation a graph can record).
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        KVHP_HIP(hipStreamIsCapturing(s, &st), "hipStreamIsCapturing(noalloc)");
        KVHP_REQUIRE(st == hipStreamCaptureStatusNone, KVHP_ERR_INVALID,
                     "decode_attention_noalloc: the first call on device %d is under graph "
                     "capture; make one call outside capture first", dev);
        void* p = nullptr;
        KVHP_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return KVHP_OK;
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
    // Rows are addressed with 32-bit byte offsets inside a 16-row page.
    if (v.stride_d != 1 || v.stride_s % 8 != 0 || v.stride_s <= 0 || v.stride_s >= (1 << 26) ||
        !aligned16(v.data))
        return false;
    if (v.block_table) return v.page_size == kPage && v.stride_h % 8 == 0;
    return v.stride_b % 8 == 0 && v.stride_h % 8 == 0;
}


// Split-kernel workgroups (one wave each) resident on the device at once.
template <typename K>
int resident_splits(K kernel) {
    return resident_workgroups(reinterpret_cast<const void*>(kernel), kWave);
}

template <int D, int G, bool TOUT>
void launch_fast(const DecodeArgs& args, dim3 grid, bool paged, hipStream_t s) {
    DecodeArgs a = args;
    if (a.balance > 0) {
        // Balanced splits: about one split per resident wave slot over the
        // batch, less half a split per sequence for the rounding up of each
        // sequence's split count.
        const int slots = paged ? resident_splits(decode_splitk_kernel<D, G, true, 1, TOUT>)
                                : resident_splits(decode_splitk_kernel<D, G, false, 1>);
        a.balance = slots > 0 ? max(1, slots / a.Hkv - a.batch / 2) : 0;
        if (a.balance > 0) {
            // Work list of every split of the batch per kv head.  The split
            // target is at least keys / balance, or max_chunk when clamped,
            // so sequence b has at most L_b / target + 1 splits and the batch
            // at most max(balance, B * cap / max_chunk) + B.
            const long long worst = ((long long)a.batch * a.cap + a.max_chunk - 1) / a.max_chunk;
            const long long units = std::max<long long>(a.balance, worst) + a.batch;
            if (units <= 65535)   // grid y limit; beyond it the fixed chunk serves
                grid = dim3(a.Hkv, static_cast<unsigned>(units), 1);
            else
                a.balance = 0;
        }
    }
    if (a.balance > 0) {   // the work list: one wave per split
        if (paged)
            hipLaunchKernelGGL((decode_splitk_kernel<D, G, true, 1, TOUT>), grid, dim3(kWave), 0, s, a);
        else
            hipLaunchKernelGGL((decode_splitk_kernel<D, G, false, 1>), grid, dim3(kWave), 0, s, a);
    } else if (D == 64 || a.nsplit == 1) {   // fixed chunks: four waves per split
        if (paged)
            hipLaunchKernelGGL((decode_splitk_kernel<D, G, true, 4, TOUT>), grid, dim3(4 * kWave), 0, s, a);
        else
            hipLaunchKernelGGL((decode_splitk_kernel<D, G, false, 4>), grid, dim3(4 * kWave), 0, s, a);
    } else {
        if (paged)
            hipLaunchKernelGGL((decode_splitk_kernel<D, G, true, 1, TOUT>), grid, dim3(kWave), 0, s, a);
        else
            hipLaunchKernelGGL((decode_splitk_kernel<D, G, false, 1>), grid, dim3(kWave), 0, s, a);
    }
    // fixed chunks with >= 64 KB of partials per (kv head, sequence): one
    // merge workgroup per query head (config 2 at 64K: 50.2 vs 51.2 us;
    // below that, e.g. config 5's 38 KB, the per-kv-head merge is faster)
    const bool rows_merge =
        a.balance <= 0 && (long long)a.nsplit * G * (D + 2) * sizeof(float) >= (64 << 10);
    if (a.nsplit > 1 && rows_merge)
        hipLaunchKernelGGL((decode_merge_rows_kernel<D, TOUT>), dim3(a.Hq, a.batch),
                           dim3(kMergeWaves * kWave), 0, s, a);
    else if (a.nsplit > 1)
        hipLaunchKernelGGL((decode_merge_kernel<D, G, TOUT>), dim3(a.Hkv, a.batch),
                           dim3(kMergeWaves * kWave), 0, s, a);
}

// A row-tiled output on paged views only (the model runner's pools).
template <int D, int G>
void launch_out(const DecodeArgs& a, dim3 grid, bool paged, hipStream_t s) {
    if (a.out_tiles > 0 && paged)
        launch_fast<D, G, true>(a, grid, paged, s);
    else
        launch_fast<D, G, false>(a, grid, paged, s);
}

template <int D>
bool dispatch_g(int G, const DecodeArgs& a, dim3 grid, bool paged, hipStream_t s) {
    switch (G) {
        case 1: launch_out<D, 1>(a, grid, paged, s); return true;
        case 2: launch_out<D, 2>(a, grid, paged, s); return true;
        case 3: launch_out<D, 3>(a, grid, paged, s); return true;
        case 4: launch_out<D, 4>(a, grid, paged, s); return true;
        case 5: launch_out<D, 5>(a, grid, paged, s); return true;
        case 6: launch_out<D, 6>(a, grid, paged, s); return true;
        case 7: launch_out<D, 7>(a, grid, paged, s); return true;
        case 8: launch_out<D, 8>(a, grid, paged, s); return true;
        case 16: launch_out<D, 16>(a, grid, paged, s); return true;
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
// k_new != nullptr: fused append (paged or strided views) -- row b of
// k_new / v_new [B][Hkv][D] goes to position new_pos[b] before attention.
int decode_attention_impl(const void* q, const kvhp_kv_view* kv, const kvhp_kv_view* vv,
                          const int32_t* seq_lens, int fixed_len, void* out, int batch,
                          int hq, int hkv, int d, int max_seq_len, int num_splits,
                          void* workspace, size_t workspace_bytes, hipStream_t s,
                          const void* k_new = nullptr, const void* v_new = nullptr,
                          const int32_t* new_pos = nullptr, int out_tiles = 0) {
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
    a.k_new = nullptr;
    a.v_new = nullptr;
    a.new_pos = nullptr;
    a.pool_k = const_cast<f16*>(static_cast<const f16*>(kv->data));
    a.pool_v = const_cast<f16*>(static_cast<const f16*>(vv->data));
    a.out_tiles = out_tiles;

    // The fast kernel reads one block table for K and V (one page id per
    // token position, the layout PagedKVCache builds).
    const bool shared_table = !paged || (kv->block_table == vv->block_table &&
                                         kv->max_pages == vv->max_pages &&
                                         kv->num_pages == vv->num_pages);
    const Plan plan = plan_for(batch, hkv, max_seq_len, num_splits, paged);
    const bool fast = (d == 64 || d == 128) && fast_group(G) && view_fast_ok(*kv) &&
                      view_fast_ok(*vv) && aligned16(q) && aligned16(out) && shared_table &&
                      plan.nsplit <= kMaxSplits;
    if (k_new) {
        KVHP_REQUIRE(v_new && new_pos, KVHP_ERR_INVALID,
                     "append_decode: k_new, v_new and positions required");
        if (fast && aligned16(k_new) && aligned16(v_new)) {
            a.k_new = static_cast<const f16*>(k_new);
            a.v_new = static_cast<const f16*>(v_new);
            a.new_pos = new_pos;
        } else if (paged) {
            // outside the fused kernel's shapes: the append, then attention
            rc = kvhp_paged_append_kv(k_new, v_new, const_cast<void*>(kv->data),
                                      const_cast<void*>(vv->data), kv->block_table,
                                      kv->max_pages, new_pos, batch, 1, hkv, d, kv->num_pages,
                                      s);
            if (rc) return rc;
        } else {
            const int64_t n = (int64_t)batch * hkv * d;
            hipLaunchKernelGGL(append_rows_strided_kernel, dim3((unsigned)((n + 255) / 256)),
                               dim3(256), 0, s, static_cast<const f16*>(k_new),
                               static_cast<const f16*>(v_new), to_dev(*kv), to_dev(*vv), new_pos,
                               batch, hkv, d, max_seq_len,
                               const_cast<f16*>(static_cast<const f16*>(kv->data)),
                               const_cast<f16*>(static_cast<const f16*>(vv->data)));
            rc = check_launch("append_decode");
            if (rc) return rc;
        }
    }
    if (!fast) {
        // Single pass: every sequence fully, no workspace.
        a.ws_o = nullptr;
        a.ws_ml = nullptr;
        a.chunk = max_seq_len;
        a.nsplit = 1;
        a.batch = batch;
        a.balance = 0;
        a.min_chunk = 0;
        a.max_chunk = max_seq_len;
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

    a.chunk = plan.chunk;
    a.nsplit = plan.nsplit;
    a.cap = plan.nsplit * plan.chunk;
    if (a.cap > max_seq_len) a.cap = max_seq_len;
    // Never address block-table columns past max_pages.
    if (paged) a.cap = min(a.cap, min(kv->max_pages, vv->max_pages) * kPage);
    // Auto split count for a batch (8 or more sequences): per-sequence
    // chunks balanced over the batch on the device (the lengths are device
    // data), within the plan's nsplit slots; a chunk may then grow up to the
    // paged limit (one page id per lane).  Config 3 (B=32, L ~ U[128, 8192]):
    // 84.4 vs 90.7 us.  Smaller batches keep the fixed chunk: the work list
    // puts the lengths' load in front of the page-table load, which cost
    // B=1 decode 1.5-2 us, and one sequence's splits are equal anyway.  An
    // explicit split count keeps the fixed chunk: exactly that split.
    a.batch = batch;
    a.balance = num_splits <= 0 && batch >= 8 ? 1 : 0;   // unit count set per kernel at launch
    // Fewest keys per split: 64 from 16 sequences, 128 below (the config-5
    // batched runner at ctx 2K with 64: B = 32 1.365 vs 1.384 ms per step,
    // B = 8 0.986 vs 0.974 ms; config 3's splits are longer either way).
    a.min_chunk = batch >= 16 ? 64 : 128;
    a.max_chunk = paged ? kMaxPagedChunk : (a.cap + kPage - 1) / kPage * kPage;
    if (a.max_chunk < plan.chunk) a.max_chunk = plan.chunk;
    const size_t need = workspace_bytes_for(batch, hq, hkv, d, plan);
    a.ws_o = nullptr;
    a.ws_ml = nullptr;
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
        const size_t ob = sizeof(float) * (size_t)batch * hq * plan.nsplit * d;
        a.ws_o = reinterpret_cast<float*>(base);
        a.ws_ml = reinterpret_cast<float*>(base + ob);
    }
    dim3 grid(plan.nsplit, hkv, batch);
    const bool ok = d == 64 ? dispatch_g<64>(G, a, grid, paged, s)
                            : dispatch_g<128>(G, a, grid, paged, s);
    if (!ok) return fail(KVHP_ERR_UNSUPPORTED, "decode_attention: group size %d", G);
    return check_launch("decode_attention");
}

int decode_attention_act(const void* q, const kvhp_kv_view* k_view, const kvhp_kv_view* v_view,
                         const int32_t* seq_lens, void* out, int batch, int num_q_heads,
                         int num_kv_heads, int head_dim, int max_seq_len, void* workspace,
                         size_t workspace_bytes, int act_tiles, hipStream_t s) {
    KVHP_REQUIRE(seq_lens && k_view && k_view->block_table, KVHP_ERR_INVALID,
                 "decode_attention_act: paged views and seq_lens required");
    KVHP_REQUIRE(act_tiles == act_tiles_for(batch) && (int64_t)num_q_heads * head_dim % 32 == 0 &&
                     aligned16(out),
                 KVHP_ERR_INVALID, "decode_attention_act: %d output tiles for batch %d, Hq*D=%d",
                 act_tiles, batch, num_q_heads * head_dim);
    return decode_attention_impl(q, k_view, v_view, seq_lens, 0, out, batch, num_q_heads,
                                 num_kv_heads, head_dim, max_seq_len, 0, workspace,
                                 workspace_bytes, s, nullptr, nullptr, nullptr, act_tiles);
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
    // the larger of the strided and the paged plan (a paged split is capped
    // at kMaxPagedChunk tokens, which can mean more splits)
    const size_t strided = workspace_bytes_for(batch, num_q_heads, num_kv_heads, head_dim,
                                               plan_for(batch, num_kv_heads, max_seq_len, num_splits, false));
    const size_t paged = workspace_bytes_for(batch, num_q_heads, num_kv_heads, head_dim,
                                             plan_for(batch, num_kv_heads, max_seq_len, num_splits, true));
    return strided > paged ? strided : paged;
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

extern "C" int kvhp_decode_attention_noalloc(const void* q, const kvhp_kv_view* k_view,
                                             const kvhp_kv_view* v_view,
                                             const int32_t* seq_lens, void* out, int batch,
                                             int num_q_heads, int num_kv_heads, int head_dim,
                                             int max_seq_len, int num_splits, void* stream) {
    clear_error();
    KVHP_REQUIRE(seq_lens, KVHP_ERR_INVALID, "decode_attention_noalloc: null seq_lens");
    KVHP_REQUIRE(k_view && v_view, KVHP_ERR_INVALID, "decode_attention_noalloc: null view");
    if (batch <= 0 || max_seq_len <= 0) return KVHP_OK;
    // the split partials of the plan this call will run, against the scratch
    const bool paged = k_view->block_table != nullptr;
    const size_t need = workspace_bytes_for(
        batch, num_q_heads, num_kv_heads, head_dim,
        plan_for(batch, num_kv_heads, max_seq_len, num_splits, paged));
    KVHP_REQUIRE(need <= kScratchBytes, KVHP_ERR_WORKSPACE,
                 "decode_attention_noalloc: %zu bytes of split partials needed, the static "
                 "scratch holds %zu (use kvhp_decode_attention with a workspace)",
                 need, kScratchBytes);
    void* ws = nullptr;
    const int rc = scratch_address(&ws, static_cast<hipStream_t>(stream));
    if (rc) return rc;
    return decode_attention_impl(q, k_view, v_view, seq_lens, 0, out, batch, num_q_heads,
                                 num_kv_heads, head_dim, max_seq_len, num_splits, ws,
                                 kScratchBytes, static_cast<hipStream_t>(stream));
}

extern "C" int kvhp_paged_append_decode(const void* q, const void* k_new, const void* v_new,
                                        const kvhp_kv_view* k_view, const kvhp_kv_view* v_view,
                                        const int32_t* positions, const int32_t* seq_lens,
                                        void* out, int batch, int num_q_heads, int num_kv_heads,
                                        int head_dim, int max_seq_len, int num_splits,
                                        void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    KVHP_REQUIRE(seq_lens && k_new && v_new && positions && k_view && v_view, KVHP_ERR_INVALID,
                 "append_decode: null pointer");
    KVHP_REQUIRE(k_view->block_table && v_view->block_table, KVHP_ERR_INVALID,
                 "append_decode: paged views required");
    return decode_attention_impl(q, k_view, v_view, seq_lens, 0, out, batch, num_q_heads,
                                 num_kv_heads, head_dim, max_seq_len, num_splits, workspace,
                                 workspace_bytes, static_cast<hipStream_t>(stream), k_new, v_new,
                                 positions);
}

extern "C" int kvhp_append_decode(const void* q, const void* k_new, const void* v_new,
                                  const kvhp_kv_view* k_view, const kvhp_kv_view* v_view,
                                  const int32_t* positions, const int32_t* seq_lens, void* out,
                                  int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                  int max_seq_len, int num_splits, void* workspace,
                                  size_t workspace_bytes, void* stream) {
    clear_error();
    KVHP_REQUIRE(seq_lens && k_new && v_new && positions && k_view && v_view, KVHP_ERR_INVALID,
                 "append_decode: null pointer");
    return decode_attention_impl(q, k_view, v_view, seq_lens, 0, out, batch, num_q_heads,
                                 num_kv_heads, head_dim, max_seq_len, num_splits, workspace,
                                 workspace_bytes, static_cast<hipStream_t>(stream), k_new, v_new,
                                 positions);
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
