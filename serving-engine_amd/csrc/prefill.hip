// prefill.hip -- causal flash attention for prefill on CDNA4 fp16 MFMA (gfx950).
//
// Work decomposition: a 512-thread workgroup (8 waves) owns one KV head and
// a query block of 32*RB rows for all G query heads of that KV head: G*RB
// units of (head, 32 rows).  With KG = 1 each wave owns one unit (RB = 8/G);
// with KG = 2 (G <= 4; chosen where doubling the workgroup count fills the
// CUs without adding a round, e.g. S <= 2048 at B = 1) two wave groups share
// the units and split every tile's keys.  Each 64-key K/V
// tile is read from HBM once per workgroup and consumed by all 8 waves, so
// GQA heads share their K/V traffic.  Query blocks i and N-1-i are processed
// by the same workgroup (two passes), giving every workgroup the same causal
// work (KG = 2: odd KV heads run the long block first), when those
// pairs fill the GPU; below that (S < 2048 at 32/8 heads) every block gets
// its own workgroup, longest first, so that more CUs share the work (S=512
// 15.4 vs 21.5 us).  Grid x enumerates (pair or block, kv_head) with the kv
// head fastest.
//
// K/V staging: a 4-stage LDS ring (4 x 32 KB for D=128), filled by
// global_load_lds_dwordx4 (direct HBM->LDS, no VGPR round trip).  Tile t+2 is
// issued when tile t's phases begin; before reading a stage each wave waits
// for its own loads of that stage (explicit s_waitcnt vmcnt(N)) and the
// workgroup meets at one barrier per ping-pong phase.  Rows are stored with an XOR
// swizzle of their 16-byte chunks so that both the K reads (ds_read_b128)
// and the transposing V reads (ds_read_b64_tr_b16) are bank-conflict free.
//
// Per tile and unit, on v_mfma_f32_32x32x16_f16, transposed so that one lane
// owns one query row for the whole online softmax:
//   S^T = K Q^T     A = K rows from LDS, B = Q^T held in registers.
//   softmax         fp32 in the log2 domain; the causal mask is applied only on
//                   tiles that cross the diagonal; the running max moves (and
//                   O is rescaled) only when a row's max passes it by 8 in
//                   log2 units, so P <= 256 stays exact in fp16; row sums by
//                   v_dot2_f32_f16 over the fp16 P.
//   O^T += V^T P^T  A = V^T read with ds_read_b64_tr_b16 (transposing 8-byte
//                   LDS reads), B = P^T converted to fp16 straight from the
//                   S^T accumulators.
// The tile loop is a ping-pong: waves 0-3 and 4-7 (one of each per SIMD)
// alternate an MFMA step (S^T of tile j, O^T of tile j-1, operand reads
// scheduled ahead, at wave priority 1) and a softmax step one phase apart.
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
constexpr int kNumCUs = 256;  // MI355X compute units (work-split heuristic only)

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
    int paired;             // 1: query blocks i and n-1-i share a workgroup (two passes)
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

// Same with a wave-uniform base in SGPRs and a 32-bit per-lane byte offset.
__device__ __forceinline__ void dma16s(const f16* sbase, uint32_t voff, f16* lds_base) {
    const uint32_t m0v = static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((lds_void*)(lds_f16*)lds_base));
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :: "s"(m0v), "v"(voff), "s"(sbase) : "memory", "m0");
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

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr float kLazyLog2 = 8.f;  // P stays below 2^8 between rescales

// Sum / max across the two 32-lane halves of a wave (v_permlane32_swap).
__device__ __forceinline__ float halves_max(float x) {
    auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(t[0]), __uint_as_float(t[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
    auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(t[0]) + __uint_as_float(t[1]);
}

// A workgroup of 8 waves serves one KV head and a query block of 32*RB rows
// for all G query heads of that KV head: G*RB units of (head, 32 rows).  With
// KG = 1 each wave owns one unit (G*RB <= 8); with KG = 2 (G <= 4) the waves
// form two groups of four that share the units and split every 64-key tile
// (group y takes keys 32y..32y+31), and the two softmax states of a unit are
// merged through LDS at the end -- half the query rows per workgroup, so
// twice the workgroups.  K/V tiles of 64 keys stream through a 4-stage LDS ring
// filled by direct global->LDS loads and are read by every wave, so GQA
// heads share their K/V traffic; rows are stored XOR-swizzled (16-byte
// chunk c of row r at position c ^ swz(r)) so the operand reads hit distinct
// banks without padding.  Query blocks i and N-1-i run in the same workgroup
// so every workgroup does the same causal work.
//
// Contractions on v_mfma_f32_32x32x16_f16 (lane l: row/column l%32, k-slots
// 8(l/32)..+8; accumulator element i is row 8(i/4) + 4(l/32) + i%4):
//   S^T = K Q^T     A = K rows (ds_read_b128), B = Q^T in registers; lane l
//                   owns query row l%32 of its unit, 32 of the 64 keys.
//   O^T += V^T P^T  per 16-key step t: A = V^T by two transposing 8-byte
//                   reads, B = P^T = fp16 of accumulator elements 8u..8u+7
//                   of key block t/2 (u = t%2): k-slot (h, e) is key
//                   16t + 4h + e for e < 4 and 16t + 8 + 4h + e - 4 above.
// Per 64-key tile a wave does 32 MFMAs (1 MFLOP) for 32 KB of LDS reads,
// twice the work per LDS byte of 16x16 tiles.
template <int D, int KG>
__global__ void __launch_bounds__(8 * kWave)
prefill_mfma_kernel(const PrefillArgs a) {
    constexpr int WAVES = 8;
    constexpr int UPG = WAVES / KG;     // units per wave group
    constexpr int NTH = WAVES * kWave;  // threads per workgroup
    constexpr int NC = D / 16;          // k-chunks of the QK contraction
    constexpr int NDB = D / 32;         // 32-dim blocks of the output
    constexpr int CPR = D / 8;          // 16-byte chunks per row
    constexpr int RPI = kWave / CPR;    // rows per DMA instruction
    constexpr int IPW = kBN / RPI / WAVES;  // DMA instructions per wave per matrix
    constexpr int LPT = 2 * IPW;        // DMA loads per wave per tile (K + V)
    constexpr int TB = kBN * D;         // halfs per tile matrix
    constexpr int KSW = CPR - 1;        // K swizzle: c ^ (r & KSW)
    // V swizzle: the transposing reads of one half-wave touch 4 consecutive
    // rows x 4 chunks; these land on distinct 16-byte bank groups of the
    // 256-byte bank line.
    auto vswz = [](int r) { return CPR == 16 ? 4 * (r & 3) : (r & 3) << 1; };

    constexpr int NSTAGE = 4;
    __shared__ __attribute__((aligned(16))) f16 ring[NSTAGE * 2 * TB];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS bases in SGPRs
    const int lane = tid & 63;
    const int h = lane >> 5;        // k-slot half
    const int c32 = lane & 31;      // row / column in the 32x32 operands
    const int j16 = lane & 15;      // lane within its 16-lane block
    const int blk2 = (lane >> 4) & 1;

    const int kvh = blockIdx.x % a.Hkv;
    const int pair = blockIdx.x / a.Hkv;   // pair index (paired) or block rank, longest first
    const int b = blockIdx.y;
    const int S = a.S;
    const int G = a.G;
    const int RB = a.RB;
    const int BM = 32 * RB;
    const int nunits = G * RB;
    const int64_t qrs = (int64_t)a.Hq * D;     // q/out row stride
    const int64_t kvrs = (int64_t)a.Hkv * D;   // k/v row stride
    const f16* kb = a.k + (int64_t)b * S * kvrs + (int64_t)kvh * D;
    const f16* vb = a.v + (int64_t)b * S * kvrs + (int64_t)kvh * D;

    // DMA of tile tt into a stage: this wave's rows (wave*IPW + p)*RPI + lane/CPR.
    // Tiles past the last one re-load the last tile (an L2 hit): every path
    // issues the same loads, so the vmcnt bookkeeping stays exact.
    // Per-lane DMA source offsets inside a tile (bytes): row and swizzled chunk.
    uint32_t dko[IPW], dvo[IPW];
#pragma unroll
    for (int p = 0; p < IPW; ++p) {
        const int row = (wave * IPW + p) * RPI + lane / CPR;
        const int ck = (lane % CPR) ^ (row & KSW);
        const int cv = (lane % CPR) ^ vswz(row);
        dko[p] = static_cast<uint32_t>((row * kvrs + 8 * ck) * 2);
        dvo[p] = static_cast<uint32_t>((row * kvrs + 8 * cv) * 2);
    }
    int last_tile = 0;
    auto issue = [&](f16* stg, int tt) {
        tt = min(tt, last_tile);
        const int key0 = tt * kBN;
        if (key0 + kBN <= S) {
            const f16* kt = kb + (int64_t)key0 * kvrs;
            const f16* vt = vb + (int64_t)key0 * kvrs;
#pragma unroll
            for (int p = 0; p < IPW; ++p) {
                const int blk = wave * IPW + p;
                dma16s(kt, dko[p], stg + blk * RPI * D);
                dma16s(vt, dvo[p], stg + TB + blk * RPI * D);
            }
        } else {
            // the last, partial tile: rows past the prompt re-read row S-1
#pragma unroll
            for (int p = 0; p < IPW; ++p) {
                const int blk = wave * IPW + p;
                const int row = blk * RPI + lane / CPR;
                const int key = min(key0 + row, S - 1);
                const int ck = (lane % CPR) ^ (row & KSW);
                const int cv = (lane % CPR) ^ vswz(row);
                dma16(kb + (int64_t)key * kvrs + 8 * ck, stg + blk * RPI * D);
                dma16(vb + (int64_t)key * kvrs + 8 * cv, stg + TB + blk * RPI * D);
            }
        }
    };
    // Per-lane LDS read offsets (halfs) inside a stage: K operand chunk c of
    // key row 32*kgrp + c32 (+32 per extra key block), and V^T operand of dim
    // block db at key row 32*kgrp + 4h + j16/4 (+16 per key step, +8 for the
    // second read).  The swizzles depend on the lane only.
    const int kgrp_ = wave / (WAVES / KG);
    int kro[NC], vro[NDB];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int r = 32 * kgrp_ + c32;
        kro[c] = r * D + 8 * ((2 * c + h) ^ (r & KSW));
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
        const int R1 = 32 * kgrp_ + 4 * h + j16 / 4;
        const int ch = 4 * db + 2 * blk2 + ((j16 & 3) >> 1);
        vro[db] = R1 * D + 8 * (ch ^ vswz(R1)) + 4 * (j16 & 1);
    }

    for (int pass = 0; pass < 2; ++pass) {
        // KG = 2: odd KV heads (other XCDs) take their long block
        // first, so that half the workgroups load Q and drain stores while
        // the other half run tile loops (every workgroup of a KV head still
        // walks the same tiles together).
        const bool flip = KG == 2 && (kvh & 1) != 0;
        int qblk;
        if (a.paired) {
            qblk = (pass == 0) != flip ? pair : a.n_qblk - 1 - pair;
            if (pass == 1 && a.n_qblk - 1 - pair <= pair) break;   // odd count: middle block once
        } else {
            if (pass == 1) break;
            qblk = a.n_qblk - 1 - pair;   // one block per workgroup, longest first
        }
        const int q0 = qblk * BM;

        // ---- this wave's unit: head kvh*G + u%G, rows r0 .. r0+31; its key
        //      half of every tile (all 64 keys when KG == 1)
        const int u = wave % UPG;
        const int kgrp = wave / UPG;
        const bool uvalid = u < nunits;
        const int qh = kvh * G + (uvalid ? u % G : 0);
        const int r0 = q0 + 32 * (uvalid ? u / G : 0);
        const int row = r0 + c32;
        half8 qop[NC];
        {
            const bool live = uvalid && row < S;
            const f16* qp = a.q + ((int64_t)b * S + row) * qrs + (int64_t)qh * D + 8 * h;
#pragma unroll
            for (int c = 0; c < NC; ++c) qop[c] = live ? load_half8(qp + 16 * c) : half8{};
        }
        floatx16 o[NDB];
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[db][i] = 0.f;
        float m_run = -1e30f, l_part = 0.f;
        const float lazy_thr = kLazyLog2 / a.scale_log2;   // in raw score units

        const int last_row = min(q0 + BM, S) - 1;
        const int n_tiles = last_row / kBN + 1;
        last_tile = n_tiles - 1;

        wait_vmcnt<0>();  // q in registers before the ring: no compiler waits inside it
        ring_barrier();   // everyone is done with the previous pass's stages
        issue(ring, 0);
        issue(ring + 2 * TB, 1);

        constexpr int NKB = 2 / KG;     // this wave's 32-key blocks per tile
        auto qk = [&](const f16* Kt, floatx16 (&sc)[NKB]) {
#pragma unroll
            for (int kb2 = 0; kb2 < NKB; ++kb2) {
#pragma unroll
                for (int i = 0; i < 16; ++i) sc[kb2][i] = 0.f;
#pragma unroll
                for (int c = 0; c < NC; ++c) {
                    const half8 kop = *reinterpret_cast<const half8*>(&Kt[kro[c] + 32 * kb2 * D]);
                    sc[kb2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kop, qop[c], sc[kb2], 0, 0, 0);
                }
            }
        };
        floatx16 sc[NKB];
        half8 pop[2 * NKB];
#pragma unroll
        for (int kb2 = 0; kb2 < NKB; ++kb2)
#pragma unroll
            for (int i = 0; i < 16; ++i) sc[kb2][i] = 0.f;
#pragma unroll
        for (int t = 0; t < 2 * NKB; ++t) pop[t] = half8{};

        // Ping-pong: the two wave groups (waves 0-3, 4-7; one wave of each per
        // SIMD; with KG = 2 the two key halves of every tile) alternate an
        // MFMA step and a softmax step, group 1 one phase behind group 0, so
        // that one wave's MFMAs run under the other's exponentials.  The
        // barriers order memory only, so the compiler may still move a step's
        // ALU work across them; the MFMA step's operand reads are scheduled PF
        // ahead of their MFMAs.  With the MFMA step at wave priority 1 this
        // beats a plain per-tile loop (QK of tile t+1, softmax of t, PV of t in
        // every wave) at every size: S=2048 45.4 vs 47.1 us, S=8192 516 vs
        // 540 us.
        //   mstep(j): S^T(j) = K(j) Q^T (j < n),  O^T += V(j-1)^T P(j-1)^T (j >= 1)
        //   sstep(j): P(j) from S^T(j); O, l rescaled when the max moves.
        // Phase 2j: group 0 mstep(j), group 1 sstep(j-1); phase 2j+1: group 0
        // sstep(j), group 1 mstep(j); one workgroup barrier between phases.
        // Ring: tile j+2 is issued at the start of phase 2j into the stage
        // of tile j-2, whose last reader (group 1's mstep(j-1)) ran in phase
        // 2j-1; before the barrier into phase 2j each wave waits for its own
        // DMA of tile j (tile j+1 may stay in flight).  Tiles past the end
        // re-load the last tile, so every wave issues the same loads.
        auto pv = [&](int j) {
            const f16* Vt = ring + (j % NSTAGE) * 2 * TB + TB;
#pragma unroll
            for (int t = 0; t < 2 * NKB; ++t) {
#pragma unroll
                for (int db = 0; db < NDB; ++db) {
                    const f16* p1 = &Vt[vro[db] + 16 * t * D];
                    const half8 vop = cat_half8(lds_read_tr16(p1), lds_read_tr16(p1 + 8 * D));
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vop, pop[t], o[db], 0, 0, 0);
                }
            }
        };
        // Operand reads run PF reads ahead of the MFMAs that use them.
        constexpr int NQK = NKB * NC, NPV = 2 * NKB * NDB;   // MFMAs
        constexpr int PF = 8;
        // The MFMA step runs at wave priority 1: when the SIMD's other wave
        // (softmax step) and this one both can issue, the MFMAs go first
        // (S=8192 516 vs 524 us, S=2048 45.4 vs 47.2 us).
        auto mstep = [&](int j) {   // 1 <= j < n_tiles
            __builtin_amdgcn_s_setprio(1);
            qk(ring + (j % NSTAGE) * 2 * TB, sc);
            pv(j - 1);
            __builtin_amdgcn_sched_group_barrier(0x100, PF, 0);
#pragma unroll
            for (int i = 0; i < NQK - PF; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
#pragma unroll
            for (int i = 0; i < NPV; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, NQK + NPV - (NQK - PF) - NPV, 0);
            __builtin_amdgcn_s_setprio(0);
        };
        auto sstep = [&](int j) {
            const int k0 = j * kBN;
            const bool act = uvalid && k0 <= r0 + 31;
            // ---- online softmax of query row `row`; P^T operands straight
            // from S^T.  Inactive units (invalid, or entirely above the
            // diagonal) see only -inf scores: alpha = 1 and p = 0 leave their
            // state as is.  The running max is kept on raw scores and the
            // scale folded into the exponent.
            if (!act || k0 + kBN - 1 > r0) {
                // element (kb2, i) holds key k0 + 32(kb2 + kgrp) + 4h +
                // 8(i/4) + i%4; keys past min(row, S-1) are masked
                const int lim = act ? min(row, S - 1) - (k0 + 32 * kgrp + 4 * h) : -1;
#pragma unroll
                for (int kb2 = 0; kb2 < NKB; ++kb2)
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (32 * kb2 + 8 * (i / 4) + (i % 4) > lim) sc[kb2][i] = -INFINITY;
            }
            float tmax = -INFINITY;
#pragma unroll
            for (int kb2 = 0; kb2 < NKB; ++kb2)
#pragma unroll
                for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, sc[kb2][i]);
            tmax = halves_max(tmax);
            // Lazy rescale: m_run is a reference max, moved (and O, l
            // rescaled) only when some row's max exceeds it by more than
            // kLazyLog2 in log2 units; otherwise p = 2^(s*c - m_run*c) stays
            // below 2^kLazyLog2, exact in fp16.
            if (__builtin_amdgcn_read_exec() & __ballot(tmax > m_run + lazy_thr)) {
                const float mn = fmaxf(m_run, tmax);
                const float alpha = fast_exp2((m_run - mn) * a.scale_log2);
                l_part *= alpha;
#pragma unroll
                for (int db = 0; db < NDB; ++db) o[db] *= alpha;
                m_run = mn;
            }
            const float nmc = -m_run * a.scale_log2;
#pragma unroll
            for (int t = 0; t < 2 * NKB; ++t)
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    pop[t][e] = static_cast<f16>(
                        fast_exp2(fmaf(sc[t / 2][8 * (t % 2) + e], a.scale_log2, nmc)));
            // Row sum of the fp16 P actually fed to the PV contraction, two
            // values per v_dot2_f32_f16 with fp32 accumulation.
            const half2v ones = {static_cast<f16>(1.f), static_cast<f16>(1.f)};
#pragma unroll
            for (int t = 0; t < 2 * NKB; ++t)
#pragma unroll
                for (int e = 0; e < 8; e += 2)
                    l_part = __builtin_amdgcn_fdot2(half2v{pop[t][e], pop[t][e + 1]}, ones, l_part,
                                                    false);
        };
        auto phase_start = [&](int j) {   // barrier into phase 2j, then tile j+2
            wait_vmcnt<LPT>();
            ring_barrier();
            const int tt = j + 2;
            issue(ring + (tt % NSTAGE) * 2 * TB, tt);
        };
        if ((wave >> 2) == 0) {
            phase_start(0);
            qk(ring, sc);
            ring_barrier();
            sstep(0);
            for (int j = 1; j < n_tiles; ++j) {
                phase_start(j);
                mstep(j);
                ring_barrier();
                sstep(j);
            }
            phase_start(n_tiles);
            pv(n_tiles - 1);
            ring_barrier();
        } else {
            phase_start(0);
            ring_barrier();
            qk(ring, sc);
            for (int j = 1; j < n_tiles; ++j) {
                phase_start(j);
                sstep(j - 1);
                ring_barrier();
                mstep(j);
            }
            phase_start(n_tiles);
            sstep(n_tiles - 1);
            ring_barrier();
            pv(n_tiles - 1);
        }
        wait_vmcnt<0>();  // drain the ring's trailing re-loads

        // ---- pages: this query block's own K/V rows, once per KV head.  Rows
        //      of the pass's last tile come from its ring stage (still intact:
        //      the trailing re-loads go to the other stages), earlier rows
        //      (blocks longer than a tile) from memory.
        if (a.pool_k) {
            const int lt0 = last_tile * kBN;
            const f16* Ks = ring + (last_tile % NSTAGE) * 2 * TB;
            const f16* Vs = Ks + TB;
            for (int idx = tid; idx < BM * CPR; idx += NTH) {
                const int key = q0 + idx / CPR;
                const int ch = idx % CPR;
                if (key >= S || key / kPage >= a.max_pages) continue;
                const int pid = a.bt[(int64_t)b * a.max_pages + key / kPage];
                if (pid < 0 || pid >= a.num_pages) continue;
                const int64_t dst =
                    (((int64_t)kvh * a.num_pages + pid) * kPage + key % kPage) * D + 8 * ch;
                half8 kk, vv;
                if (key >= lt0) {
                    const int r = key - lt0;
                    kk = *reinterpret_cast<const half8*>(&Ks[r * D + 8 * (ch ^ (r & KSW))]);
                    vv = *reinterpret_cast<const half8*>(&Vs[r * D + 8 * (ch ^ vswz(r))]);
                } else {
                    kk = load_half8(kb + (int64_t)key * kvrs + 8 * ch);
                    vv = load_half8(vb + (int64_t)key * kvrs + 8 * ch);
                }
                store_half8(a.pool_k + dst, kk);
                store_half8(a.pool_v + dst, vv);
            }
        }

        if constexpr (KG == 2) {
            // ---- group 1 hands its (m, l, O) to group 0 through the ring's
            //      LDS (every wave is past its last read of the ring).
            float* xo = reinterpret_cast<float*>(ring);
            float* xml = xo + UPG * NDB * 16 * kWave;
            ring_barrier();
            if (kgrp == 1) {
#pragma unroll
                for (int db = 0; db < NDB; ++db)
#pragma unroll
                    for (int q4 = 0; q4 < 4; ++q4) {
                        floatx4 v4 = {o[db][4 * q4], o[db][4 * q4 + 1], o[db][4 * q4 + 2],
                                      o[db][4 * q4 + 3]};
                        *reinterpret_cast<floatx4*>(
                            &xo[(((u * NDB + db) * 4 + q4) * kWave + lane) * 4]) = v4;
                    }
                xml[(u * kWave + lane) * 2] = m_run;
                xml[(u * kWave + lane) * 2 + 1] = l_part;
            }
            ring_barrier();
            if (kgrp == 0) {
                const float m1 = xml[(u * kWave + lane) * 2];
                const float l1 = xml[(u * kWave + lane) * 2 + 1];
                const float mn = fmaxf(m_run, m1);
                const float a0 = fast_exp2((m_run - mn) * a.scale_log2);
                const float a1 = fast_exp2((m1 - mn) * a.scale_log2);
                l_part = l_part * a0 + l1 * a1;
#pragma unroll
                for (int db = 0; db < NDB; ++db)
#pragma unroll
                    for (int q4 = 0; q4 < 4; ++q4) {
                        const floatx4 v4 = *reinterpret_cast<const floatx4*>(
                            &xo[(((u * NDB + db) * 4 + q4) * kWave + lane) * 4]);
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            o[db][4 * q4 + e] = o[db][4 * q4 + e] * a0 + v4[e] * a1;
                    }
            }
        }

        // ---- normalise and store: lane holds row `row`, dims 32db + 8q + 4h + e.
        {
            const float lt = halves_sum(l_part);
            if (kgrp == 0 && uvalid && row < S) {
                const float inv = lt > 0.f ? 1.f / lt : 0.f;
                f16* orow = a.out + ((int64_t)b * S + row) * qrs + (int64_t)qh * D + 4 * h;
#pragma unroll
                for (int db = 0; db < NDB; ++db)
#pragma unroll
                    for (int q4 = 0; q4 < 4; ++q4) {
                        half4 hv;
#pragma unroll
                        for (int e = 0; e < 4; ++e) hv[e] = static_cast<f16>(o[db][4 * q4 + e] * inv);
                        *reinterpret_cast<half4*>(orow + 32 * db + 8 * q4) = hv;
                    }
            }
        }

        wait_vmcnt<0>();   // page and output stores complete before the next ring starts
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
    a.paired = 1;

    const bool fast = (d == 64 || d == 128) && a.G <= 8 && aligned16(q) && aligned16(k) &&
                      aligned16(v) && aligned16(out) &&
                      (!pool_k || (aligned16(pool_k) && aligned16(pool_v)));
    if (fast) {
        // units of (head, 32 rows) per workgroup: one per wave, or (G <= 4)
        // one per pair of waves that split each tile's keys (KG = 2: twice
        // the workgroups, each with half the rows).  A KG = 2 workgroup takes
        // ~57 % of a KG = 1 workgroup's time, so KG = 2 pays when doubling
        // the workgroups adds no round of CUs: with grid1 block pairs of one
        // unit per wave, up to half the CUs (grid1 <= 128) or one and a half
        // rounds (257..384).  Measured at 32/8 heads, D = 128: KG = 1 is
        // 12-32 % faster at grid1 = 144..256 (S = 2304..4096 at B = 1,
        // S = 1280..2048 at B = 2), 10 % at 448 and 8 % at 512; KG = 2 is
        // 19 % faster at 128 (S = 2048) and 1-10 % at 288..384.
        const int64_t qblk1 = (seq_len + 32 * (8 / a.G) - 1) / (32 * (8 / a.G));
        const int64_t grid1 = (int64_t)hkv * ((qblk1 + 1) / 2) * batch;
        const bool split = grid1 <= kNumCUs / 2 || (grid1 > kNumCUs && grid1 <= kNumCUs * 3 / 2);
        const int kg = ((a.G == 1 || a.G == 2 || a.G == 4) && split) ? 2 : 1;
        a.RB = 8 / kg / a.G;
        const int bm = 32 * a.RB;
        a.n_qblk = static_cast<int>((seq_len + bm - 1) / bm);
        // pair the causal blocks only when the pairs fill every CU
        const int64_t pgrid = (int64_t)hkv * ((a.n_qblk + 1) / 2) * batch;
        a.paired = (pgrid >= kNumCUs) ? 1 : 0;
        dim3 grid(hkv * (a.paired ? (a.n_qblk + 1) / 2 : a.n_qblk), batch);
        const dim3 blk(8 * kWave);
        if (d == 64 && kg == 2)
            hipLaunchKernelGGL((prefill_mfma_kernel<64, 2>), grid, blk, 0, s, a);
        else if (d == 64)
            hipLaunchKernelGGL((prefill_mfma_kernel<64, 1>), grid, blk, 0, s, a);
        else if (kg == 2)
            hipLaunchKernelGGL((prefill_mfma_kernel<128, 2>), grid, blk, 0, s, a);
        else
            hipLaunchKernelGGL((prefill_mfma_kernel<128, 1>), grid, blk, 0, s, a);
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
