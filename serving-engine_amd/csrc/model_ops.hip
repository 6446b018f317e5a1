// model_ops.hip -- operators of the decoder-only model around the KV-cache
// path (config 5: Llama-style 1.1B, batch-1 greedy decode), for gfx950.
//
// Decode (one token) is HBM-bound on the weights: every projection is a
// GEMV y = W x with W fp16 [N][K] row-major, read once.  A wave owns RW
// output rows; lane l holds the 16-byte chunks 512j + 8l .. +8 of x in
// registers for the whole kernel and streams the same chunks of its rows
// (RW*K/512 non-temporal 16-byte loads in flight per lane), multiplies with
// v_dot2_f32_f16 (fp16 products, fp32 accumulation) and reduces each row
// across the wave with DPP + row swaps.  The neighbouring element-wise work
// of the reference's decode step is fused into that kernel:
//   prologue  RMSNorm of x (sum of squares in fp32, x*rsqrt*w rounded to
//             fp16 as the reference's norm_out buffer, rmsnorm.cu:16-70);
//   epilogue  fp16 store, residual add (gemv_residual, gemv.cu), fp32 logits,
//             SwiGLU of a gate row and its up row (swiglu.cu; the gate and up
//             values are rounded to fp16 first, as the reference's separate
//             GEMV outputs are), or RoPE + KV-cache append for the fused QKV
//             projection (rope.cu:8-57 then kv_cache.cu:8-36: q/k rounded to
//             fp16, rotated in fp32, rounded again; k and v written into their
//             16-token pages at position seq_len - 1).
// A generic one-wave-per-row kernel covers shapes the fast one does not.
//
// Prefill uses library GEMMs (rocBLAS) for the projections; the row-wise
// RMSNorm, the RoPE that also splits the fused QKV output, and SwiGLU over
// the fused gate|up output are here.  Greedy sampling is an on-device argmax
// with the lowest index winning ties (the reference's host loop,
// generate.cpp:714-721), which also advances the device-side sequence length
// so that a captured decode step needs no host round trip.
#include "kvhp_internal.h"

#include <algorithm>
#include <cmath>

namespace kvhp {

namespace {


constexpr int kNumCUs = 256;  // MI355X compute units (tile-size heuristic only)

enum Epilogue : int { kEpiF16 = 0, kEpiResidual = 1, kEpiF32 = 2, kEpiSwiglu = 3, kEpiQKV = 4 };

struct GemvArgs {
    const f16* W;          // [rows][K]
    const f16* x;          // [K]
    const f16* norm_w;     // [K] RMSNorm weight (prologue), or null
    float eps;
    int N;                 // output rows (SwiGLU: gate rows, up rows follow)
    int K;
    f16* y16;              // fp16 output
    float* y32;            // fp32 output
    const f16* resid;      // residual added in the epilogue (may alias y16)
    // fused QKV: rows [Hq*D q | Hkv*D k | Hkv*D v]
    int Hq, Hkv, D;
    const int32_t* seq_len;  // device: the token is at position seq_len[0] - len_offset
    int len_offset;          // 1: seq_len holds the bumped length; 0: it holds the position
    float theta;
    f16* pool_k;           // [Hkv][num_pages][16][D]
    f16* pool_v;
    const int32_t* bt;     // block table of the sequence [max_pages]
    int max_pages, num_pages;
};

__device__ __forceinline__ float dot8(half8 a, half8 b, float acc) {
    acc = __builtin_amdgcn_fdot2(half2v{a[0], a[1]}, half2v{b[0], b[1]}, acc, false);
    acc = __builtin_amdgcn_fdot2(half2v{a[2], a[3]}, half2v{b[2], b[3]}, acc, false);
    acc = __builtin_amdgcn_fdot2(half2v{a[4], a[5]}, half2v{b[4], b[5]}, acc, false);
    acc = __builtin_amdgcn_fdot2(half2v{a[6], a[7]}, half2v{b[6], b[7]}, acc, false);
    return acc;
}

__device__ __forceinline__ float round16(float v) { return static_cast<float>(static_cast<f16>(v)); }

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.f + expf(-g)) * u; }

// RoPE angle of dimension pair i (< D/2) at position pos, as the reference
// computes it in float (ops.cpp:174-186).
__device__ __forceinline__ void rope_cs(int pos, int i, int D, float theta, float& c, float& s) {
    const float inv = 1.f / powf(theta, static_cast<float>(2 * i) / static_cast<float>(D));
    const float ang = static_cast<float>(pos) * inv;
    c = cosf(ang);
    s = sinf(ang);
}

// Fast GEMV: K == 512*KC, RW rows per wave (one wave per workgroup).
template <int KC, int RW, int EPI, bool RMS>
__global__ void __launch_bounds__(kWave) gemv_kernel(const GemvArgs a) {
    const int lane = threadIdx.x;

    // The rows of this wave.
    int row[RW];
    bool ok[RW];
    const int wv = blockIdx.x;
    if constexpr (EPI == kEpiQKV) {
        // head hh, pair block pb: rows hh*D + (RW/2)pb + i and
        // hh*D + D/2 + (RW/2)pb + i, i < RW/2
        const int wph = a.D / RW;
        const int hh = wv / wph, pb = wv % wph;
#pragma unroll
        for (int i = 0; i < RW; ++i) {
            row[i] = hh * a.D + (i < RW / 2 ? 0 : a.D / 2) + (RW / 2) * pb + (i % (RW / 2));
            ok[i] = true;
        }
    } else if constexpr (EPI == kEpiSwiglu) {
#pragma unroll
        for (int i = 0; i < RW; ++i) {
            const int n = wv * (RW / 2) + (i % (RW / 2));
            ok[i] = n < a.N;
            row[i] = (ok[i] ? n : 0) + (i < RW / 2 ? 0 : a.N);
        }
    } else {
#pragma unroll
        for (int i = 0; i < RW; ++i) {
            const int n = wv * RW + i;
            ok[i] = n < a.N;
            row[i] = ok[i] ? n : 0;
        }
    }

    // Weights, x and the norm weights are independent: every load is issued
    // before the first use, so the wave makes one memory round trip (the
    // scheduler would otherwise interleave loads and products to save
    // registers, and the RMSNorm would serialise two more trips).  x and the
    // norm weights go first: vector loads complete in issue order, so the
    // RMSNorm waits only for them and runs while the weights stream in
    // (behind the weights it waited for every weight load: QKV 4.25 vs
    // 3.58 us without the norm, in a HIP graph).
    half8 xr[KC], nw[KC];
#pragma unroll
    for (int j = 0; j < KC; ++j) {
        xr[j] = load_half8(a.x + 512 * j + 8 * lane);
        if constexpr (RMS) nw[j] = load_half8(a.norm_w + 512 * j + 8 * lane);
    }
    __builtin_amdgcn_sched_barrier(0);   // keep them ahead of the weights
    half8 wr[RW][KC];
#pragma unroll
    for (int i = 0; i < RW; ++i)
#pragma unroll
        for (int j = 0; j < KC; ++j)
            wr[i][j] = load_half8_stream(a.W + (int64_t)row[i] * a.K + 512 * j + 8 * lane);
    // The epilogue's own reads (residual row, write position and its page)
    // ride the same round trip.
    float rv = 0.f;
    if constexpr (EPI == kEpiResidual) {
        int rr = row[0];
#pragma unroll
        for (int i = 1; i < RW; ++i)
            if (lane == i) rr = row[i];
        rv = static_cast<float>(a.resid[rr]);
    }
    int pos = 0, pid = -1;
    float rc = 1.f, rs = 0.f;  // RoPE rotation of this lane's pair
    if constexpr (EPI == kEpiQKV) {
        pos = a.seq_len[0] - a.len_offset;
        if (pos >= 0 && (pos >> 4) < a.max_pages) pid = a.bt[pos >> 4];
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (EPI == kEpiQKV) {
        // The angle depends only on the position and the pair: computed here,
        // under the weight loads, instead of after the products.
        const int hh = wv / (a.D / RW);
        if (hh < a.Hq + a.Hkv) {
            rope_cs(pos < 0 ? 0 : pos, (RW / 2) * (wv % (a.D / RW)) + lane, a.D, a.theta, rc, rs);
            asm volatile("" ::"v"(rc), "v"(rs));
        }
    }
    if constexpr (RMS) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < KC; ++j)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float v = static_cast<float>(xr[j][e]);
                ss = fmaf(v, v, ss);
            }
        ss = wave_sum_fast(ss);
        const float rs = 1.f / sqrtf(ss / static_cast<float>(a.K) + a.eps);
#pragma unroll
        for (int j = 0; j < KC; ++j)
#pragma unroll
            for (int e = 0; e < 8; ++e)
                xr[j][e] = static_cast<f16>(static_cast<float>(xr[j][e]) * rs *
                                            static_cast<float>(nw[j][e]));
    }
    float acc[RW];
#pragma unroll
    for (int i = 0; i < RW; ++i) {
        acc[i] = 0.f;
#pragma unroll
        for (int j = 0; j < KC; ++j) acc[i] = dot8(wr[i][j], xr[j], acc[i]);
        acc[i] = wave_sum_fast(acc[i]);
    }

    // Lane i (< RW) finishes row i (every lane holds every sum).
    if constexpr (EPI == kEpiQKV) {
        if (lane >= RW / 2) return;
        float x1 = 0.f, x2 = 0.f;
#pragma unroll
        for (int i = 0; i < RW / 2; ++i)
            if (lane == i) {
                x1 = round16(acc[i]);
                x2 = round16(acc[RW / 2 + i]);
            }
        const int wph = a.D / RW;
        const int hh = wv / wph, pb = wv % wph;
        const int d = (RW / 2) * pb + lane;   // pair (d, d + D/2)
        const int half = a.D / 2;
        if (hh >= a.Hq + a.Hkv) {             // v: no rotation
            const int kvh = hh - a.Hq - a.Hkv;
            if (pid < 0 || pid >= a.num_pages) return;
            f16* dst = a.pool_v + (((int64_t)kvh * a.num_pages + pid) * kPage + (pos & 15)) * a.D;
            dst[d] = static_cast<f16>(x1);
            dst[d + half] = static_cast<f16>(x2);
            return;
        }
        const float c = rc, s = rs;
        const f16 o1 = static_cast<f16>(x1 * c - x2 * s);
        const f16 o2 = static_cast<f16>(x2 * c + x1 * s);
        if (hh < a.Hq) {
            a.y16[hh * a.D + d] = o1;
            a.y16[hh * a.D + d + half] = o2;
        } else {
            const int kvh = hh - a.Hq;
            if (pid < 0 || pid >= a.num_pages) return;
            f16* dst = a.pool_k + (((int64_t)kvh * a.num_pages + pid) * kPage + (pos & 15)) * a.D;
            dst[d] = o1;
            dst[d + half] = o2;
        }
    } else if constexpr (EPI == kEpiSwiglu) {
        if (lane >= RW / 2) return;
        float g = 0.f, u = 0.f;
        bool valid = false;
        int n = 0;
#pragma unroll
        for (int i = 0; i < RW / 2; ++i)
            if (lane == i) {
                g = round16(acc[i]);
                u = round16(acc[RW / 2 + i]);
                valid = ok[i];
                n = row[i];
            }
        if (valid) a.y16[n] = static_cast<f16>(silu_mul(g, u));
    } else {
        if (lane >= RW) return;
        float v = 0.f;
        bool valid = false;
        int n = 0;
#pragma unroll
        for (int i = 0; i < RW; ++i)
            if (lane == i) {
                v = acc[i];
                valid = ok[i];
                n = row[i];
            }
        if (!valid) return;
        if constexpr (EPI == kEpiF32) {
            a.y32[n] = v;
        } else if constexpr (EPI == kEpiResidual) {
            a.y16[n] = static_cast<f16>(v + rv);
        } else {
            a.y16[n] = static_cast<f16>(v);
        }
    }
}

// Generic GEMV: one wave per output row (SwiGLU: per gate/up pair; QKV: per
// rotation pair), any K.  RMSNorm prologue recomputed by every wave.
template <int EPI, bool RMS>
__global__ void __launch_bounds__(kWave) gemv_generic_kernel(const GemvArgs a) {
    const int lane = threadIdx.x;
    float rs = 1.f;
    if constexpr (RMS) {
        float ss = 0.f;
        for (int k = lane; k < a.K; k += kWave) {
            const float v = static_cast<float>(a.x[k]);
            ss = fmaf(v, v, ss);
        }
        ss = wave_sum_fast(ss);
        rs = 1.f / sqrtf(ss / static_cast<float>(a.K) + a.eps);
    }
    auto xin = [&](int k) {
        if constexpr (RMS)
            return static_cast<float>(static_cast<f16>(static_cast<float>(a.x[k]) * rs *
                                                       static_cast<float>(a.norm_w[k])));
        else
            return static_cast<float>(a.x[k]);
    };
    auto dot_row = [&](int r) {
        float acc = 0.f;
        const f16* w = a.W + (int64_t)r * a.K;
        for (int k = lane; k < a.K; k += kWave) acc = fmaf(static_cast<float>(w[k]), xin(k), acc);
        return wave_sum_fast(acc);
    };
    const int t = blockIdx.x;
    if constexpr (EPI == kEpiQKV) {
        const int half = a.D / 2;
        const int hh = t / half, d = t % half;
        const float x1 = round16(dot_row(hh * a.D + d));
        const float x2 = round16(dot_row(hh * a.D + d + half));
        if (lane != 0) return;
        const int pos = a.seq_len[0] - a.len_offset;
        float o1 = x1, o2 = x2;
        if (hh < a.Hq + a.Hkv) {
            float c, s;
            rope_cs(pos < 0 ? 0 : pos, d, a.D, a.theta, c, s);
            o1 = x1 * c - x2 * s;
            o2 = x2 * c + x1 * s;
        }
        if (hh < a.Hq) {
            a.y16[hh * a.D + d] = static_cast<f16>(o1);
            a.y16[hh * a.D + d + half] = static_cast<f16>(o2);
            return;
        }
        if (pos < 0 || (pos >> 4) >= a.max_pages) return;
        const int pid = a.bt[pos >> 4];
        if (pid < 0 || pid >= a.num_pages) return;
        const bool isk = hh < a.Hq + a.Hkv;
        const int kvh = isk ? hh - a.Hq : hh - a.Hq - a.Hkv;
        f16* dst = (isk ? a.pool_k : a.pool_v) +
                   (((int64_t)kvh * a.num_pages + pid) * kPage + (pos & 15)) * a.D;
        dst[d] = static_cast<f16>(o1);
        dst[d + half] = static_cast<f16>(o2);
    } else if constexpr (EPI == kEpiSwiglu) {
        const float g = round16(dot_row(t));
        const float u = round16(dot_row(a.N + t));
        if (lane == 0) a.y16[t] = static_cast<f16>(silu_mul(g, u));
    } else {
        const float v = dot_row(t);
        if (lane != 0) return;
        if constexpr (EPI == kEpiF32)
            a.y32[t] = v;
        else if constexpr (EPI == kEpiResidual)
            a.y16[t] = static_cast<f16>(v + static_cast<float>(a.resid[t]));
        else
            a.y16[t] = static_cast<f16>(v);
    }
}

template <int EPI, bool RMS>
int launch_gemv(const GemvArgs& a, hipStream_t s) {
    int units;  // rows (or row pairs) the generic kernel runs one wave each on
    if constexpr (EPI == kEpiQKV)
        units = (a.Hq + 2 * a.Hkv) * (a.D / 2);
    else
        units = a.N;
    const bool xa = aligned16(a.x) && aligned16(a.W) && (!RMS || aligned16(a.norm_w));
    // Two rows per wave: the decode GEMVs are latency-bound, and more, smaller
    // waves in flight beat fewer that each stream more rows (measured on the
    // config-5 step: 1448 tok/s at 2 rows, 1430 at 4, 1376 at 8).
    if (xa && a.K == 2048) {
        constexpr int RW = 2;
        int grid;
        if constexpr (EPI == kEpiQKV)
            grid = (a.Hq + 2 * a.Hkv) * (a.D / RW);
        else if constexpr (EPI == kEpiSwiglu)
            grid = (a.N + RW / 2 - 1) / (RW / 2);
        else
            grid = (a.N + RW - 1) / RW;
        hipLaunchKernelGGL((gemv_kernel<4, RW, EPI, RMS>), dim3(grid), dim3(kWave), 0, s, a);
    } else if (xa && a.K == 5632 && EPI != kEpiQKV && EPI != kEpiSwiglu) {
        constexpr int RW = 2;
        hipLaunchKernelGGL((gemv_kernel<11, RW, EPI, RMS>), dim3((a.N + RW - 1) / RW),
                           dim3(kWave), 0, s, a);
    } else {
        hipLaunchKernelGGL((gemv_generic_kernel<EPI, RMS>), dim3(units), dim3(kWave), 0, s, a);
    }
    return check_launch("gemv");
}

// Workgroup barrier that orders LDS only: this wave's LDS reads and writes
// complete (lgkmcnt(0)) before s_barrier, and its global loads stay in
// flight.  __syncthreads() would also wait for every outstanding global load:
// the weights the MFMAs need next and the next tile's prefetch.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0); vmcnt and expcnt left free
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// ---- Batched decode projections (B <= 32 sequences per step) -----------------
// Y[b][n] = sum_k W[n][k] X[b][k] on v_mfma_f32_16x16x32_f16 with the weights
// as the A operand.  A tile is 16 weight rows; for the paired epilogues its
// first 8 rows pair with its last 8 (SwiGLU: gate rows n..n+7 with up rows
// N+n..N+n+7; RoPE: dims d..d+7 with d+D/2..d+D/2+7 of one head).  The NW
// waves of a workgroup split K into slices of 32*C (slice s: k in
// [32Cs, 32C(s+1)), wave w taking slice (w + rot) % NW with rot chosen per
// workgroup) and keep their slice of X (all B rows: NBT tiles of 16,
// zero past B; RMSNorm applied once) in registers, while the workgroup walks
// tiles blockIdx.x, +gridDim.x, ... (grid = the resident workgroups): the
// next tile's weights are loaded before the current tile's MFMAs, and the
// epilogue's own reads (residual) before those, so each wave keeps a tile of
// loads in flight while it computes and reduces.  Lane (g, col) = (l/16,
// l%16) loads row col of a tile at k = 32t + 8g (16 bytes; an instruction
// reads 64 contiguous bytes of 16 rows) and the same k of batch row col; the
// accumulator holds D[4g + e][col].  The NW partial tiles meet in LDS (two
// buffers, one barrier per tile) and are summed in slice order
// (deterministic), then the batch-1 GEMV's epilogue runs per (row, batch
// row).  RMSNorm: the waves' sums of squares of their slices meet in LDS
// first, so the operand is fp16(x * rs * w) as the batch-1 kernel rounds it.
struct RowsArgs {
    const f16* W;          // [rows][K]
    const f16* Wt;         // the same weights tiled (rows_tile_kernel), or null: loads
                           // then read 1 KB contiguous per wave and k step
    const f16* x;          // [B][K]
    const f16* norm_w;     // [K] RMSNorm weight, or null
    float eps;
    int N, K, B;
    int tiles;             // weight tiles
    int live;              // distinct weight rows per tile: 16, or 8 when tiles are
                           // scarce (lanes past it repeat rows; their outputs are dropped)
    // (on the first 64-byte line of the arguments, with W, x and the sizes)
    int x_tiles;           // > 0: x row-tiled (act_tiled_index, this many batch tiles)
    int y_tiles;           // > 0: y16 and resid row-tiled (residual / SwiGLU epilogues)
    f16* y16;              // [B][ldy] (QKV: q [B][Hq*D])
    float* y32;            // [B][ldy]
    const f16* resid;      // [B][ldy], may alias y16
    int ldy;
    int Hq, Hkv, D;
    const int32_t* positions;  // [B] write position of each row (QKV); < 0: idle row
    float theta;
    f16* pool_k;           // [Hkv][num_pages][16][D]
    f16* pool_v;
    const int32_t* bt;     // [B][max_pages]
    int max_pages, num_pages;
};

template <int C, int NWMAX, int NBT, int EPI, bool RMS>
__global__ void __launch_bounds__(kWave * NWMAX) gemm_rows_kernel(const RowsArgs a) {
    constexpr bool kPair = EPI == kEpiSwiglu || EPI == kEpiQKV;
    constexpr int kOut = 256;                 // (row, column) slots per batch tile and weight tile
    const int L = a.live, P = a.live / 2;     // live rows; row pairs (paired epilogues)
    // Past ~128 VGPRs (16 waves per workgroup) x is not kept: each tile loads
    // its batch tiles in turn into one set of registers, and the weights are
    // not double-buffered.
    constexpr bool kSeq = !RMS && NBT > 1 && (1 + NBT) * C * 4 > 120;
    // Two weight buffers where the registers allow (8-wave workgroups);
    // otherwise each tile loads its weights at its start.
    constexpr bool kDB = !kSeq && (NWMAX <= 8 || (2 + NBT) * C * 4 <= 100);
    // 256-wide slices (K <= 2048): each wave stages its x slice through its
    // own LDS region with contiguous loads (512 bytes of a row per 32 lanes),
    // then reads it back in the MFMA layout.  Loaded directly in that layout
    // (16 rows of 64 bytes, 4 KB apart, per instruction) the same bytes took
    // 4.7 us per launch at B = 32 against 3.4 us staged (2.5 us read
    // linearly, 1.6 us for an empty launch).
    constexpr bool kStage = !kSeq && C == 8;
    constexpr int kCH = 4 * C;                           // 16-byte chunks per slice row
    constexpr int kRedBytes = 2 * NBT * 256 * 4;         // a wave's two partial-sum buffers
    constexpr int kStgBytes = kStage ? NBT * 16 * kCH * 16 : 0;
    constexpr int kWaveBytes = kRedBytes > kStgBytes ? kRedBytes : kStgBytes;
    // per wave: the x stage, then (once x is in registers) the partial sums
    __shared__ __attribute__((aligned(16))) char lds[NWMAX * kWaveBytes];
    __shared__ float ssq[NBT][NWMAX][16];
    auto red = [&](int rb, int wi, int bt) {
        return reinterpret_cast<float*>(lds + wi * kWaveBytes) + (rb * NBT + bt) * 256;
    };
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int NW = static_cast<int>(blockDim.x >> 6);
    const int g = lane >> 4, col = lane & 15;
    // Wave w holds K slice (w + rot) % NW: the workgroups of one XCD
    // (blockIdx.x equal mod 8) start their x loads on different slices
    // instead of all reading the same lines at once.  Partial sums are
    // still added in slice order, so results do not depend on rot.
    const int rot = static_cast<int>((blockIdx.x >> 3) % static_cast<unsigned>(NW));
    const int sl = w + rot < NW ? w + rot : w + rot - NW;
    const int ks = sl * 32 * C + 8 * g;
    const int G = static_cast<int>(gridDim.x);
    const int n_my = (a.tiles - static_cast<int>(blockIdx.x) + G - 1) / G;

    auto load_w = [&](int tile, half8 (&wr)[C]) {
        int row;
        const int j = col % L;   // live row of this lane
        if constexpr (EPI == kEpiQKV) {
            const int tph = a.D / L;
            const int hh = tile / tph, d0 = P * (tile % tph);
            row = hh * a.D + (j < P ? 0 : a.D / 2) + d0 + (j % P);
        } else if constexpr (EPI == kEpiSwiglu) {
            const int n = min(P * tile + (j % P), a.N - 1);
            row = j < P ? n : a.N + n;
        } else {
            row = min(L * tile + j, a.N - 1);
        }
        const f16* wp = a.W + (int64_t)row * a.K + ks;
        // lanes past the live rows load nothing (their output rows are dropped)
        if (col < L && a.Wt) {
            // tiled: 16-row tiles (paired epilogues always run 16 live rows on
            // them); 8 live rows are half h of tile tile/2 (plain rows only)
            const int t16 = L == 16 ? tile : tile >> 1;
            const int l = L == 16 ? lane : 16 * g + 8 * (tile & 1) + col;
            const f16* tp = a.Wt + (((int64_t)t16 * (a.K / 32) + sl * C) * kWave + l) * 8;
#pragma unroll
            for (int t = 0; t < C; ++t) wr[t] = load_half8_stream(tp + t * kWave * 8);
        } else if (col < L) {
#pragma unroll
            for (int t = 0; t < C; ++t) wr[t] = load_half8_stream(wp + 32 * t);
        } else {
#pragma unroll
            for (int t = 0; t < C; ++t) wr[t] = half8{};
        }
    };
    auto load_x = [&](int bt, half8 (&xs)[C]) {
        const int b = 16 * bt + col;   // columns past B: zero, not loaded
        if (a.x_tiles) {   // row-tiled: k step (slice, t) of batch tile bt, 1 KB per wave
#pragma unroll
            for (int t = 0; t < C; ++t)
                xs[t] = load_half8(a.x + ((((int64_t)sl * C + t) * a.x_tiles + bt) * kWave + lane) * 8);
        } else if (b < a.B) {
#pragma unroll
            for (int t = 0; t < C; ++t) xs[t] = load_half8(a.x + (int64_t)b * a.K + ks + 32 * t);
        } else {
#pragma unroll
            for (int t = 0; t < C; ++t) xs[t] = half8{};
        }
    };

    // fp16 output / residual element (b, n): row-major with pitch ldy, or row-tiled
    auto yat = [&](int b, int n) -> int64_t {
        return a.y_tiles ? act_tiled_index(b, n, a.y_tiles) : (int64_t)b * a.ldy + n;
    };

    half8 wa[C], wb[C];
    int tile = static_cast<int>(blockIdx.x);
    if constexpr (kSeq) {
        if constexpr (kDB) load_w(tile, wa);
    }

    // x slice of every batch tile, resident for all tiles (RMSNorm applied)
    half8 xr[kSeq ? 1 : NBT][C];
    if constexpr (!kSeq) {
        // staged: lane i of load j takes chunk (64j + i) % kCH of slice row
        // (64j + i) / kCH; rows past B load nothing (zero)
        constexpr int kNL = kStage ? NBT * 16 * kCH / kWave : 1;
        half8 stg[kNL];
        if (kStage && a.x_tiles == 0) {
            const f16* xs0 = a.x + sl * 32 * C;
#pragma unroll
            for (int j = 0; j < kNL; ++j) {
                const int idx = j * kWave + lane, row = idx / kCH, ch = idx % kCH;
                stg[j] = row < a.B ? load_half8(xs0 + (int64_t)row * a.K + 8 * ch) : half8{};
            }
        } else {
            // row-tiled x (any C), or row-major x outside the staged shapes
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt) load_x(bt, xr[bt]);
        }
        half8 nw[C];
        if constexpr (RMS) {
#pragma unroll
            for (int t = 0; t < C; ++t) nw[t] = load_half8(a.norm_w + ks + 32 * t);
        }
        // the first tile's weights after x: the RMSNorm below waits for x
        // only, the weights keep landing under it
        if constexpr (kDB) load_w(tile, wa);
        // every load above in flight before the first use (one round trip;
        // the scheduler would otherwise pair loads with their uses)
        __builtin_amdgcn_sched_barrier(0);
        if (kStage && a.x_tiles == 0) {
            // into this wave's region (chunk c of row r at c ^ (r & 7): the
            // 8-lane phases of both the writes and the operand reads hit
            // distinct banks), then back in the layout of the B operand
            half8* st = reinterpret_cast<half8*>(lds + w * kWaveBytes);
#pragma unroll
            for (int j = 0; j < kNL; ++j) {
                const int idx = j * kWave + lane, row = idx / kCH, ch = idx % kCH;
                st[row * kCH + (ch ^ (row & 7))] = stg[j];
            }
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt)
#pragma unroll
                for (int t = 0; t < C; ++t)
                    xr[bt][t] = st[(16 * bt + col) * kCH + ((g + 4 * t) ^ (col & 7))];
        }
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt)
            if (16 * bt + col >= a.B)
#pragma unroll
                for (int t = 0; t < C; ++t) xr[bt][t] = half8{};
        if constexpr (RMS) {
            // Sum of squares of the slice: fp16 pairs on v_dot2_f32_f16 into
            // four independent fp32 chains, added in a fixed order (one
            // 64-long chain of fp32 FMAs per batch tile: ~0.6 us more per
            // launch at B = 32).
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt) {
                float s4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int t = 0; t < C; ++t)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const half2v v = {xr[bt][t][2 * e], xr[bt][t][2 * e + 1]};
                        s4[e] = __builtin_amdgcn_fdot2(v, v, s4[e], false);
                    }
                float ss = (s4[0] + s4[1]) + (s4[2] + s4[3]);
                ss = rows4_sum(ss);
                if (g == 0) ssq[bt][w][col] = ss;
            }
            lds_barrier();   // the weights keep landing under the scaling below
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt) {
                float tot = 0.f;
                for (int i = 0; i < NW; ++i) tot += ssq[bt][i >= rot ? i - rot : i - rot + NW][col];
                const float rs = 1.f / sqrtf(tot / static_cast<float>(a.K) + a.eps);
                // fp16(x * rs * w) with fp32 products, as fused multiplies of
                // the fp16 operands (no separate conversions)
#pragma unroll
                for (int t = 0; t < C; ++t)
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        xr[bt][t][e] = static_cast<f16>(
                            fmaf(fmaf(static_cast<float>(xr[bt][t][e]), rs, 0.f),
                                 static_cast<float>(nw[t][e]), 0.f));
            }
        }
    }

    // This thread's first output of a tile: batch row b0 (the same for every
    // tile); for the QKV epilogue its write position and page, loaded once.
    const int o0 = static_cast<int>(threadIdx.x);
    const int b0 = 16 * (o0 / kOut) + (o0 & 15);
    int pos0 = -1, pid0 = -1;
    if constexpr (EPI == kEpiQKV) {
        if (o0 < NBT * kOut && b0 < a.B) {
            pos0 = a.positions[b0];
            if (pos0 >= 0 && (pos0 >> 4) < a.max_pages)
                pid0 = a.bt[(int64_t)b0 * a.max_pages + (pos0 >> 4)];
        }
    }

    // Output o of a tile from its reduced sums; rv: the residual of that
    // output (Residual epilogue).
    auto epilogue = [&](int tl, int o, int rb, float rv, int pos, int pid) {
        const int bt = o / kOut, rem = o % kOut, m = rem >> 4, n = rem & 15;
        const int b = 16 * bt + n;
        if (b >= a.B || m >= (kPair ? P : L)) return;
        float v0 = 0.f, v1 = 0.f;
        for (int i = 0; i < NW; ++i) {   // slice i sits in wave (i - rot) mod NW
            const int wi = i >= rot ? i - rot : i - rot + NW;
            const float* rp = red(rb, wi, bt);
            v0 += rp[m * 16 + n];
            if constexpr (kPair) v1 += rp[(m + P) * 16 + n];
        }
        if constexpr (EPI == kEpiQKV) {
            const int tph = a.D / L;
            const int hh = tl / tph, d = P * (tl % tph) + m, half = a.D / 2;
            const float x1 = round16(v0), x2 = round16(v1);
            float o1 = x1, o2 = x2;
            if (hh < a.Hq + a.Hkv) {
                float c, sn;
                rope_cs(pos < 0 ? 0 : pos, d, a.D, a.theta, c, sn);
                o1 = x1 * c - x2 * sn;
                o2 = x2 * c + x1 * sn;
            }
            if (hh < a.Hq) {
                f16* q = a.y16 + (int64_t)b * a.ldy + hh * a.D;
                q[d] = static_cast<f16>(o1);
                q[d + half] = static_cast<f16>(o2);
                return;
            }
            if (pid < 0 || pid >= a.num_pages) return;
            const bool isk = hh < a.Hq + a.Hkv;
            const int kvh = isk ? hh - a.Hq : hh - a.Hq - a.Hkv;
            f16* dst = (isk ? a.pool_k : a.pool_v) +
                       (((int64_t)kvh * a.num_pages + pid) * kPage + (pos & 15)) * a.D;
            dst[d] = static_cast<f16>(o1);
            dst[d + half] = static_cast<f16>(o2);
        } else if constexpr (EPI == kEpiSwiglu) {
            const int nn = P * tl + m;
            if (nn < a.N) a.y16[yat(b, nn)] = static_cast<f16>(silu_mul(round16(v0), round16(v1)));
        } else {
            const int nn = L * tl + m;
            if (nn >= a.N) return;
            if constexpr (EPI == kEpiF32)
                a.y32[(int64_t)b * a.ldy + nn] = v0;
            else if constexpr (EPI == kEpiResidual)
                a.y16[yat(b, nn)] = static_cast<f16>(v0 + rv);
            else
                a.y16[yat(b, nn)] = static_cast<f16>(v0);
        }
    };

    // One tile: residual read, next tile's weights (pf), MFMAs, partial sums
    // to LDS buffer rb, barrier, epilogue.
    auto step = [&](int tl, half8 (&cur)[C], half8 (&nxt)[C], int rb, bool pf) {
        f16 r0 = static_cast<f16>(0.f);
        if constexpr (EPI == kEpiResidual) {
            const int nn = min(L * tl + min((o0 % kOut) / 16, L - 1), a.N - 1);
            if (o0 < NBT * kOut && b0 < a.B) r0 = a.resid[yat(b0, nn)];
        }
        if (pf && kDB) load_w(tl + G, nxt);
        if constexpr (!kDB) load_w(tl, cur);
        __builtin_amdgcn_sched_barrier(0);
        floatx4 acc[NBT];
        if constexpr (kSeq) {
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt) {
                half8 xs[C];
                load_x(bt, xs);
                __builtin_amdgcn_sched_barrier(0);
                if (16 * bt + col >= a.B)
#pragma unroll
                    for (int t = 0; t < C; ++t) xs[t] = half8{};
                acc[bt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int t = 0; t < C; ++t)
                    acc[bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur[t], xs[t], acc[bt], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
#pragma unroll
            for (int bt = 0; bt < NBT; ++bt) {
                acc[bt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int t = 0; t < C; ++t)
                    acc[bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur[t], xr[bt][t], acc[bt], 0, 0, 0);
            }
        }
#pragma unroll
        for (int bt = 0; bt < NBT; ++bt) {
            float* rp = red(rb, w, bt);
#pragma unroll
            for (int e = 0; e < 4; ++e) rp[(4 * g + e) * 16 + col] = acc[bt][e];
        }
        // LDS-only: the next tile's weights (prefetched above) stay in flight
        // through the barrier and the epilogue
        lds_barrier();
        for (int o = o0; o < NBT * kOut; o += static_cast<int>(blockDim.x)) {
            if (o == o0) {
                epilogue(tl, o, rb, static_cast<float>(r0), pos0, pid0);
            } else {
                const int b = 16 * (o / kOut) + (o & 15);
                float rv = 0.f;
                int pos = -1, pid = -1;
                if (b < a.B) {
                    if constexpr (EPI == kEpiResidual)
                        rv = static_cast<float>(
                            a.resid[yat(b, min(L * tl + min((o % kOut) / 16, L - 1), a.N - 1))]);
                    if constexpr (EPI == kEpiQKV) {
                        pos = a.positions[b];
                        if (pos >= 0 && (pos >> 4) < a.max_pages)
                            pid = a.bt[(int64_t)b * a.max_pages + (pos >> 4)];
                    }
                }
                epilogue(tl, o, rb, rv, pos, pid);
            }
        }
    };

    // Tiles in pairs so that the two weight buffers keep fixed registers; the
    // last tile of the workgroup issues no prefetch.
    for (int i = 0;;) {
        if (i + 1 < n_my) {
            step(tile, wa, wb, 0, true);
        } else {
            step(tile, wa, wb, 0, false);
            break;
        }
        tile += G;
        ++i;
        if (i + 1 < n_my) {
            step(tile, wb, wa, 1, true);
        } else {
            step(tile, wb, wa, 1, false);
            break;
        }
        tile += G;
        ++i;
    }
}

// Slice shape for K: C = 8 (8 x 16 bytes per lane and row) with K/256 <= 8
// waves, or C = 11 with K/352 <= 16 waves (K = 5632: 16 waves).  Other K, or
// B > 32: unsupported (the caller keeps the library GEMM).
bool rows_shape(int K, int& C, int& NW) {
    if (K % 256 == 0 && K / 256 >= 1 && K / 256 <= 8) {
        C = 8;
        NW = K / 256;
        return true;
    }
    if (K % 352 == 0 && K / 352 >= 1 && K / 352 <= 16) {
        C = 11;
        NW = K / 352;
        return true;
    }
    return false;
}

template <int C, int NWMAX, int NBT, int EPI, bool RMS>
void launch_rows_k(const RowsArgs& a, int NW, hipStream_t s) {
    auto kern = gemm_rows_kernel<C, NWMAX, NBT, EPI, RMS>;
    // one workgroup per resident slot, each walking its share of the tiles
    const int slots = resident_workgroups(reinterpret_cast<const void*>(kern), kWave * NW);
    const int grid = slots > 0 ? std::min(a.tiles, slots) : a.tiles;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(kWave * NW), 0, s, a);
}

template <int C, int NWMAX, int EPI, bool RMS>
void launch_rows_c(const RowsArgs& a, int NW, hipStream_t s) {
    if (a.B <= 16)
        launch_rows_k<C, NWMAX, 1, EPI, RMS>(a, NW, s);
    else
        launch_rows_k<C, NWMAX, 2, EPI, RMS>(a, NW, s);
}

template <int EPI, bool RMS>
int launch_rows(RowsArgs a, hipStream_t s, const char* what) {
    int C = 0, NW = 0;
    KVHP_REQUIRE(a.B >= 1 && a.B <= 32, KVHP_ERR_UNSUPPORTED, "%s: batch %d outside 1..32", what,
                 a.B);
    KVHP_REQUIRE(rows_shape(a.K, C, NW), KVHP_ERR_UNSUPPORTED,
                 "%s: K=%d is neither 256*n (n <= 8) nor 352*n (n <= 16)", what, a.K);
    KVHP_REQUIRE(aligned16(a.W) && aligned16(a.x) && (!RMS || aligned16(a.norm_w)),
                 KVHP_ERR_UNSUPPORTED, "%s: W, x and the norm weight must be 16-byte aligned",
                 what);
    // 16 live rows per tile, or 8 when 16 leaves CUs idle and 8 still fits
    // one tile per CU (a second round of tiles costs more than idle CUs)
    auto tiles_for = [&](int live) {
        if constexpr (EPI == kEpiQKV)
            return (a.Hq + 2 * a.Hkv) * (a.D / live);
        else if constexpr (EPI == kEpiSwiglu)
            return (a.N + live / 2 - 1) / (live / 2);
        else
            return (a.N + live - 1) / live;
    };
    a.live = tiles_for(16) < kNumCUs && tiles_for(8) <= kNumCUs ? 8 : 16;
    if (a.Wt && (EPI == kEpiSwiglu || EPI == kEpiQKV)) a.live = 16;   // the tiles' row pairing
    a.tiles = tiles_for(a.live);
    if (C == 8) {
        launch_rows_c<8, 8, EPI, RMS>(a, NW, s);
    } else {
        if constexpr (EPI == kEpiResidual && !RMS)
            launch_rows_c<11, 16, EPI, RMS>(a, NW, s);
        else
            return fail(KVHP_ERR_UNSUPPORTED, "%s: K=%d needs the 352-wide slices, which only the "
                        "residual projection has", what, a.K);
    }
    return check_launch(what);
}

// ---- Batched residual projection split over K (large B*K) ---------------------
// Every workgroup of gemm_rows_kernel loads all B rows of x, B*K*2 bytes per
// CU (360 KB for the down projection at B = 32, more than its weights).
// Split over K instead: workgroup (row group, slice) stages the B x 32C slice
// of x in LDS once (22.5 KB at B = 32, C = 11) and its kWpg waves each
// multiply one 16-row weight tile by it, writing fp32 partial sums
// part[slice][b][n]; a second launch adds the slices in order and the
// residual.  The slices are gemm_rows_kernel's per-wave K slices and both
// sum them in slice order, so the result is bit-identical to it.
constexpr int kWpg = 8;        // weight tiles (waves) per workgroup
constexpr int kMaxSlices = 16;

template <int C, int NBT>
__global__ void __launch_bounds__(kWave * kWpg) ksplit_partial_kernel(const RowsArgs a,
                                                                      float* part) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int g = lane >> 4, col = lane & 15;
    const int slice = static_cast<int>(blockIdx.y);
    const int k0 = slice * 32 * C;
    const int tile = static_cast<int>(blockIdx.x) * kWpg + w;
    __shared__ half8 xs[NBT][16][C][4];   // [batch tile][batch row][chunk t][k group g]

    // this wave's weight tile first (streamed once; rows past N repeat row N-1)
    half8 wr[C];
    if (a.Wt) {   // tiled: tiles past the last (their outputs dropped) re-read it
        const int t16 = min(tile, (a.N + 15) / 16 - 1);
        const f16* tp = a.Wt + (((int64_t)t16 * (a.K / 32) + slice * C) * kWave + lane) * 8;
#pragma unroll
        for (int t = 0; t < C; ++t) wr[t] = load_half8_stream(tp + t * kWave * 8);
    } else {
        const int row = min(tile * 16 + col, a.N - 1);
        const f16* wp = a.W + (int64_t)row * a.K + k0 + 8 * g;
#pragma unroll
        for (int t = 0; t < C; ++t) wr[t] = load_half8_stream(wp + 32 * t);
    }
    // x slice of every batch row, zero past B; row-tiled x: the slice is one
    // contiguous run of C * NBT 1 KB blocks, copied as is ([t][bt][lane])
    half8* xsf = &xs[0][0][0][0];
    if (a.x_tiles) {
        const f16* src = a.x + (int64_t)slice * C * NBT * kWave * 8;
        for (int i = static_cast<int>(threadIdx.x); i < NBT * C * kWave; i += kWave * kWpg)
            xsf[i] = load_half8(src + (int64_t)i * 8);
    } else {
        for (int i = static_cast<int>(threadIdx.x); i < NBT * 16 * 4 * C; i += kWave * kWpg) {
            const int r = i / (4 * C), ch = i % (4 * C);   // ch = 4t + k group
            half8 v = {};
            if (r < a.B) v = load_half8(a.x + (int64_t)r * a.K + k0 + 8 * ch);
            xs[r / 16][r % 16][ch / 4][ch % 4] = v;
        }
    }
    __syncthreads();
    // this lane's operand of (batch tile bt, k step t) at xsf[xo + bt * xsb + t * xst]
    const int xo = a.x_tiles ? lane : col * C * 4 + g;
    const int xsb = a.x_tiles ? kWave : 16 * C * 4;
    const int xst = a.x_tiles ? kWave * NBT : 4;
    floatx4 acc[NBT];
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt) {
        acc[bt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < C; ++t)
            acc[bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wr[t], xsf[xo + bt * xsb + t * xst],
                                                             acc[bt], 0, 0, 0);
    }
    // lane (g, col): rows 4g..4g+3 of the tile for batch row col of each batch tile
    const int n0 = tile * 16 + 4 * g;
    if (n0 >= a.N) return;
#pragma unroll
    for (int bt = 0; bt < NBT; ++bt) {
        const int b = 16 * bt + col;
        if (b < a.B)
            *reinterpret_cast<floatx4*>(part + ((int64_t)slice * a.B + b) * a.N + n0) = acc[bt];
    }
}

// y[b][n] = fp16(sum over slices in order + resid[b][n]); 4 outputs per thread
// (resid may alias y: each element is read and written by one thread).
__global__ void __launch_bounds__(128) ksplit_reduce_residual_kernel(const RowsArgs a,
                                                                     const float* part,
                                                                     int slices) {
    const int64_t i = (int64_t)blockIdx.x * 128 + threadIdx.x;
    const int64_t total = (int64_t)a.B * a.N;
    if (i * 4 >= total) return;
    const int64_t o = i * 4;
    floatx4 p[kMaxSlices];
#pragma unroll
    for (int s = 0; s < kMaxSlices; ++s)
        p[s] = s < slices ? *reinterpret_cast<const floatx4*>(part + s * total + o)
                          : floatx4{0.f, 0.f, 0.f, 0.f};
    floatx4 v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < kMaxSlices; ++s)
        if (s < slices) v += p[s];
    const int64_t b = o / a.N, n = o % a.N;   // N % 16 == 0: the 4 outputs share a row
    // (and, row-tiled, one aligned group of 8: contiguous too)
    const int64_t y0 = a.y_tiles ? act_tiled_index(b, n, a.y_tiles) : b * a.ldy + n;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        a.y16[y0 + e] = static_cast<f16>(v[e] + static_cast<float>(a.resid[y0 + e]));
}

// Bytes of fp32 partials the K-split path needs for this call, 0 when the
// call keeps gemm_rows_kernel: batches whose x exceeds 160 KB per CU
// (B*K > 81920: the down projection, K = 5632, from B = 15), N % 16 == 0.
size_t ksplit_bytes(int N, int K, int B) {
    int C = 0, NW = 0;
    if (B < 1 || B > 32 || N % 16 != 0 || !rows_shape(K, C, NW)) return 0;
    if ((int64_t)B * K <= 81920) return 0;
    return sizeof(float) * (size_t)NW * B * N;
}

int launch_ksplit_residual(const RowsArgs& a, float* part, hipStream_t s, const char* what) {
    int C = 0, NW = 0;
    rows_shape(a.K, C, NW);
    const dim3 grid((a.N / 16 + kWpg - 1) / kWpg, NW);
    const dim3 blk(kWave * kWpg);
    if (C == 8 && a.B <= 16)
        hipLaunchKernelGGL((ksplit_partial_kernel<8, 1>), grid, blk, 0, s, a, part);
    else if (C == 8)
        hipLaunchKernelGGL((ksplit_partial_kernel<8, 2>), grid, blk, 0, s, a, part);
    else if (a.B <= 16)
        hipLaunchKernelGGL((ksplit_partial_kernel<11, 1>), grid, blk, 0, s, a, part);
    else
        hipLaunchKernelGGL((ksplit_partial_kernel<11, 2>), grid, blk, 0, s, a, part);
    const int64_t threads = (int64_t)a.B * a.N / 4;
    hipLaunchKernelGGL(ksplit_reduce_residual_kernel, dim3((unsigned)((threads + 127) / 128)),
                       dim3(128), 0, s, a, part, NW);
    return check_launch(what);
}

// ---- Tiled weights for the batched projections --------------------------------
// Tile T holds the 16 rows gemm_rows_kernel maps to lanes col = 0..15 of a
// 16-live-row tile -- plain: row 16T + col; SwiGLU: gate row n = 8T + col % 8
// (col < 8) and its up row N + n (col >= 8); QKV: dims d0 .. d0+7 of head
// T / (D/16) (col < 8) and their RoPE partners d0 + D/2 .. (col >= 8), d0 =
// 8 (T % (D/16)) -- and stores k step s (k = 32s .. 32s+31) of lane l = 16g +
// col, W[row][32s + 8g .. +8], as the 16 bytes at ((T * K/32 + s) * 64 + l) * 8
// halfs.  A wave's load of one k step is then 1 KB contiguous and a tile 32K
// bytes; row-major loads of the same operands (16 rows of 64 bytes, 4 KB
// apart, per instruction) streamed the gate/up weights at 4.2 TB/s against
// 6.0 TB/s tiled.  Rows past the matrix repeat its last row (those outputs
// are dropped), so the kernels' arithmetic and results are unchanged.
__device__ __forceinline__ int tiled_row(int kind, int N, int D, int T, int col) {
    if (kind == KVHP_ROWS_QKV) {
        const int tph = D / 16, d0 = 8 * (T % tph);
        return (T / tph) * D + (col < 8 ? 0 : D / 2) + d0 + (col & 7);
    }
    if (kind == KVHP_ROWS_SWIGLU) {
        const int n = min(8 * T + (col & 7), N - 1);
        return col < 8 ? n : N + n;
    }
    return min(16 * T + col, N - 1);
}

__global__ void __launch_bounds__(256) rows_tile_kernel(const f16* W, f16* Wt, int kind, int N,
                                                        int K, int D, int64_t chunks) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= chunks) return;
    const int l = static_cast<int>(i % kWave);
    const int64_t ts = i / kWave;
    const int s = static_cast<int>(ts % (K / 32));
    const int T = static_cast<int>(ts / (K / 32));
    const int row = tiled_row(kind, N, D, T, l & 15);
    store_half8(Wt + i * 8, load_half8(W + (int64_t)row * K + 32 * s + 8 * (l >> 4)));
}

// 16-row tiles of a tiled matrix (as gemm_rows_kernel counts them at 16 live
// rows); 0 for unsupported shapes.
int64_t rows_tiles(int kind, int N, int K, int Hq, int Hkv, int D) {
    int C = 0, NW = 0;
    if (K <= 0 || !rows_shape(K, C, NW)) return 0;
    if (kind == KVHP_ROWS_QKV)
        return Hq > 0 && Hkv > 0 && D > 0 && D % 16 == 0 ? (int64_t)(Hq + 2 * Hkv) * (D / 16) : 0;
    if (N <= 0) return 0;
    if (kind == KVHP_ROWS_SWIGLU) return (N + 7) / 8;
    if (kind == KVHP_ROWS_PLAIN) return (N + 15) / 16;
    return 0;
}

// Row-wise RMSNorm (prefill): one workgroup of 256 threads per row.
__global__ void __launch_bounds__(256)
rmsnorm_rows_kernel(const f16* x, const f16* w, f16* out, int dim, float eps) {
    __shared__ float part[4];
    const int64_t r = blockIdx.x;
    const f16* xr = x + r * dim;
    float ss = 0.f;
    for (int k = threadIdx.x; k < dim; k += 256) {
        const float v = static_cast<float>(xr[k]);
        ss = fmaf(v, v, ss);
    }
    ss = wave_sum_fast(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = part[0] + part[1] + part[2] + part[3];
    const float rs = 1.f / sqrtf(ss / static_cast<float>(dim) + eps);
    for (int k = threadIdx.x; k < dim; k += 256)
        out[r * dim + k] =
            static_cast<f16>(static_cast<float>(xr[k]) * rs * static_cast<float>(w[k]));
}

// RoPE in place on token-major q [S][Hq][D] and k [S][Hkv][D] (reference
// apply_rope, kernels.h:57-70): one thread per rotation pair.
__global__ void rope_kernel(f16* q, f16* k, int64_t S, int Hq, int Hkv, int D, int start_pos,
                            float theta) {
    const int half = D / 2;
    const int64_t pairs = S * (int64_t)(Hq + Hkv) * half;
    for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < pairs;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int i = static_cast<int>(t % half);
        const int64_t sh = t / half;
        const int h = static_cast<int>(sh % (Hq + Hkv));
        const int64_t s = sh / (Hq + Hkv);
        f16* v = h < Hq ? q + (s * Hq + h) * D : k + (s * Hkv + (h - Hq)) * D;
        float c, sn;
        rope_cs(static_cast<int>(start_pos + s), i, D, theta, c, sn);
        const float x1 = static_cast<float>(v[i]), x2 = static_cast<float>(v[i + half]);
        v[i] = static_cast<f16>(x1 * c - x2 * sn);
        v[i + half] = static_cast<f16>(x2 * c + x1 * sn);
    }
}

// Split the fused QKV projection [S][(Hq + 2Hkv) D] into contiguous q, k, v
// with RoPE applied to q and k.  Row s sits at position start_pos + s, or at
// positions[s] (device int32; negative = an idle batch row, rotated as 0)
// when positions is given.
__global__ void split_qkv_rope_kernel(const f16* qkv, int64_t S, int Hq, int Hkv, int D,
                                      int start_pos, const int32_t* positions, float theta,
                                      f16* q, f16* k, f16* v) {
    const int half = D / 2;
    const int H = Hq + 2 * Hkv;
    const int64_t pairs = S * (int64_t)H * half;
    for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < pairs;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int i = static_cast<int>(t % half);
        const int64_t sh = t / half;
        const int h = static_cast<int>(sh % H);
        const int64_t s = sh / H;
        const f16* src = qkv + (s * H + h) * D;
        const float x1 = static_cast<float>(src[i]), x2 = static_cast<float>(src[i + half]);
        f16* dst;
        float o1 = x1, o2 = x2;
        if (h < Hq + Hkv) {
            float c, sn;
            const int pos = positions ? max(positions[s], 0) : static_cast<int>(start_pos + s);
            rope_cs(pos, i, D, theta, c, sn);
            o1 = x1 * c - x2 * sn;
            o2 = x2 * c + x1 * sn;
            dst = h < Hq ? q + (s * Hq + h) * D : k + (s * Hkv + (h - Hq)) * D;
        } else {
            dst = v + (s * Hkv + (h - Hq - Hkv)) * D;
        }
        dst[i] = static_cast<f16>(o1);
        dst[i + half] = static_cast<f16>(o2);
    }
}

// SwiGLU over rows of a fused [gate | up] buffer [rows][2n] -> out [rows][n];
// with row stride 0 and n = count this is the reference's flat swiglu.
__global__ void swiglu_kernel(const f16* gate, const f16* up, int64_t in_stride, f16* out,
                              int64_t rows, int64_t n) {
    const int64_t total = rows * n;
    for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = t / n, i = t % n;
        const float g = static_cast<float>(gate[r * in_stride + i]);
        const float u = static_cast<float>(up[r * in_stride + i]);
        out[t] = static_cast<f16>(silu_mul(g, u));
    }
}

// Embedding lookup: out[i][:] = table[ids[i]][:] (ids device int32; ids
// outside [0, vocab) give zero rows).
__global__ void embedding_kernel(const int32_t* ids, const f16* table, f16* out, int64_t n,
                                 int64_t hidden, int64_t vocab) {
    const int64_t i = blockIdx.x;
    const int64_t id = ids[i];
    for (int64_t k = threadIdx.x; k < hidden; k += blockDim.x)
        out[i * hidden + k] = (id >= 0 && id < vocab) ? table[id * hidden + k] : static_cast<f16>(0.f);
}

// The same rows into row-tiled activations (hidden % 32 == 0, 16-byte
// aligned table): 8 columns per thread, contiguous in both layouts.
__global__ void embedding_tiled_kernel(const int32_t* ids, const f16* table, f16* out,
                                       int64_t hidden, int64_t vocab, int nbt) {
    const int64_t i = blockIdx.x;
    const int64_t id = ids[i];
    const bool ok = id >= 0 && id < vocab;
    for (int64_t k = 8 * threadIdx.x; k < hidden; k += 8 * blockDim.x)
        store_half8(out + act_tiled_index(i, k, nbt), ok ? load_half8(table + id * hidden + k) : half8{});
}

// Greedy argmax of fp32 logits, lowest index on ties; NaN never wins.
// Each candidate is one 64-bit key, (order-preserving bits of the value) <<
// 32 | ~index, so every reduction step is a single unsigned max: the larger
// value wins, then the smaller index; NaN maps below -inf.  Optionally
// appends the token to log[count] (count = *log_count, then incremented),
// advances *seq_len by one, and copies the token's embedding row into x
// (the next decode step's input, so that step needs no embedding launch).
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t i) {
    const uint32_t u = __float_as_uint(v);
    const uint32_t ord = (v != v) ? 0u : ((u & 0x80000000u) ? ~u : (u | 0x80000000u));
    return (static_cast<uint64_t>(ord) << 32) | static_cast<uint64_t>(~i);
}

// Workgroup r reduces row r of logits [gridDim.x][n] into token[r].
__global__ void __launch_bounds__(1024)
argmax_kernel(const float* logits, int64_t n, int32_t* token, int32_t* seq_len, int32_t* log,
              int32_t* log_count, const f16* embed, int64_t hidden, f16* x) {
    __shared__ uint64_t red[16];
    __shared__ int32_t tok_lds;
    logits += blockIdx.x * n;
    token += blockIdx.x;
    uint64_t best = 0;  // below every candidate (a NaN candidate has ~i > 0)
    // Thread t scans float4 groups t, t + 1024, ... (all of a pass's loads
    // in flight), then the scalar tail.
    const int64_t n4 = (reinterpret_cast<uintptr_t>(logits) & 15) == 0 ? n / 4 : 0;
    const floatx4* l4 = reinterpret_cast<const floatx4*>(logits);
    constexpr int U = 8;
    for (int64_t g0 = threadIdx.x; g0 < n4; g0 += (int64_t)U * blockDim.x) {
        floatx4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t g = min(g0 + (int64_t)u * blockDim.x, n4 - 1);
            v[u] = l4[g];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t g = g0 + (int64_t)u * blockDim.x;
            if (g < n4) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint64_t k = argmax_key(v[u][e], static_cast<uint32_t>(4 * g + e));
                    best = k > best ? k : best;
                }
            }
        }
    }
    for (int64_t i = 4 * n4 + threadIdx.x; i < n; i += blockDim.x) {
        const uint64_t k = argmax_key(logits[i], static_cast<uint32_t>(i));
        best = k > best ? k : best;
    }
    for (int off = 32; off >= 1; off >>= 1) {
        const uint64_t o = __shfl_xor(best, off);
        best = o > best ? o : best;
    }
    const int w = threadIdx.x >> 6;
    const int nw = static_cast<int>(blockDim.x >> 6);
    if ((threadIdx.x & 63) == 0) red[w] = best;
    __syncthreads();
    if (threadIdx.x < 64) {
        best = threadIdx.x < static_cast<unsigned>(nw) ? red[threadIdx.x] : 0;
        for (int off = 32; off >= 1; off >>= 1) {
            const uint64_t o = __shfl_xor(best, off);
            best = o > best ? o : best;
        }
        if (threadIdx.x == 0) {
            const uint32_t idx = ~static_cast<uint32_t>(best);
            const int32_t tok = best != 0 && idx < n ? static_cast<int32_t>(idx) : 0;
            *token = tok;
            tok_lds = tok;
            if (log) log[(*log_count)++] = tok;
            if (seq_len) *seq_len += 1;
        }
    }
    if (embed == nullptr) return;
    __syncthreads();
    const f16* row = embed + static_cast<int64_t>(tok_lds) * hidden;
    if ((hidden & 7) == 0 && (reinterpret_cast<uintptr_t>(row) & 15) == 0 &&
        (reinterpret_cast<uintptr_t>(x) & 15) == 0) {
        for (int64_t i = threadIdx.x; i < hidden / 8; i += blockDim.x)
            store_half8(x + 8 * i, load_half8(row + 8 * i));
    } else {
        for (int64_t i = threadIdx.x; i < hidden; i += blockDim.x) x[i] = row[i];
    }
}

// Seeded N(0, std) fill: element i of stream `stream_id` is a Box-Muller
// normal from two 64-bit splitmix hashes of (seed, stream_id, i).
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__global__ void randn_kernel(f16* out, int64_t n, uint64_t seed, uint64_t stream_id, float std) {
    const uint64_t base = splitmix64(seed ^ splitmix64(stream_id));
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const uint64_t h1 = splitmix64(base + 2 * static_cast<uint64_t>(i));
        const uint64_t h2 = splitmix64(base + 2 * static_cast<uint64_t>(i) + 1);
        const float u1 = (static_cast<float>(h1 >> 40) + 0.5f) * (1.f / 16777216.f);  // (0, 1)
        const float u2 = static_cast<float>(h2 >> 40) * (1.f / 16777216.f);          // [0, 1)
        const float r = sqrtf(-2.f * logf(u1));
        out[i] = static_cast<f16>(std * r * cospif(2.f * u2));
    }
}
__global__ void fill_kernel(f16* out, int64_t n, float value) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        out[i] = static_cast<f16>(value);
}

unsigned grid_for(int64_t n, int threads) {
    int64_t g = (n + threads - 1) / threads;
    if (g > 8192) g = 8192;
    return static_cast<unsigned>(g < 1 ? 1 : g);
}

}  // namespace

}  // namespace kvhp

using namespace kvhp;

namespace {
GemvArgs gemv_args(const void* W, const void* x, int N, int K) {
    GemvArgs a{};
    a.W = static_cast<const f16*>(W);
    a.x = static_cast<const f16*>(x);
    a.N = N;
    a.K = K;
    return a;
}
int check_gemv(const void* W, const void* x, int N, int K, const char* what) {
    KVHP_REQUIRE(W && x, KVHP_ERR_INVALID, "%s: null pointer", what);
    KVHP_REQUIRE(N > 0 && K > 0, KVHP_ERR_INVALID, "%s: N=%d K=%d must be positive", what, N, K);
    return KVHP_OK;
}
}  // namespace

extern "C" int kvhp_gemv(const void* W, const void* x, void* y, int N, int K, void* stream) {
    clear_error();
    if (N == 0) return KVHP_OK;
    int rc = check_gemv(W, x, N, K, "gemv");
    if (rc) return rc;
    KVHP_REQUIRE(y, KVHP_ERR_INVALID, "gemv: null output");
    GemvArgs a = gemv_args(W, x, N, K);
    a.y16 = static_cast<f16*>(y);
    return launch_gemv<kEpiF16, false>(a, static_cast<hipStream_t>(stream));
}

extern "C" int kvhp_gemv_residual(const void* W, const void* x, const void* r, void* y, int N,
                                  int K, void* stream) {
    clear_error();
    if (N == 0) return KVHP_OK;
    int rc = check_gemv(W, x, N, K, "gemv_residual");
    if (rc) return rc;
    KVHP_REQUIRE(r && y, KVHP_ERR_INVALID, "gemv_residual: null residual/output");
    GemvArgs a = gemv_args(W, x, N, K);
    a.resid = static_cast<const f16*>(r);
    a.y16 = static_cast<f16*>(y);
    return launch_gemv<kEpiResidual, false>(a, static_cast<hipStream_t>(stream));
}

extern "C" int kvhp_rmsnorm_gemv(const void* W, const void* x, const void* norm_w, float eps,
                                 void* y16, float* y32, int N, int K, void* stream) {
    clear_error();
    if (N == 0) return KVHP_OK;
    int rc = check_gemv(W, x, N, K, "rmsnorm_gemv");
    if (rc) return rc;
    KVHP_REQUIRE(norm_w, KVHP_ERR_INVALID, "rmsnorm_gemv: null norm weight");
    KVHP_REQUIRE((y16 != nullptr) != (y32 != nullptr), KVHP_ERR_INVALID,
                 "rmsnorm_gemv: give exactly one of y16 / y32");
    GemvArgs a = gemv_args(W, x, N, K);
    a.norm_w = static_cast<const f16*>(norm_w);
    a.eps = eps;
    a.y16 = static_cast<f16*>(y16);
    a.y32 = y32;
    hipStream_t s = static_cast<hipStream_t>(stream);
    return y32 ? launch_gemv<kEpiF32, true>(a, s) : launch_gemv<kEpiF16, true>(a, s);
}

extern "C" int kvhp_rmsnorm_gemv_swiglu(const void* W_gate_up, const void* x, const void* norm_w,
                                        float eps, void* out, int N, int K, void* stream) {
    clear_error();
    if (N == 0) return KVHP_OK;
    int rc = check_gemv(W_gate_up, x, N, K, "rmsnorm_gemv_swiglu");
    if (rc) return rc;
    KVHP_REQUIRE(norm_w && out, KVHP_ERR_INVALID, "rmsnorm_gemv_swiglu: null pointer");
    GemvArgs a = gemv_args(W_gate_up, x, N, K);
    a.norm_w = static_cast<const f16*>(norm_w);
    a.eps = eps;
    a.y16 = static_cast<f16*>(out);
    return launch_gemv<kEpiSwiglu, true>(a, static_cast<hipStream_t>(stream));
}

namespace {
// seq_len[0] - len_offset is the token's position.
int qkv_rope_append_impl(const void* W_qkv, const void* x, const void* norm_w, float eps,
                         const int32_t* seq_len, int len_offset, float rope_theta, void* q_out,
                         void* pool_k, void* pool_v, const int32_t* block_table, int max_pages,
                         int num_pages, int num_q_heads, int num_kv_heads, int head_dim, int K,
                         void* stream) {
    const int N = (num_q_heads + 2 * num_kv_heads) * head_dim;
    int rc = check_gemv(W_qkv, x, N, K, "rmsnorm_qkv_rope_append");
    if (rc) return rc;
    KVHP_REQUIRE(norm_w && seq_len && q_out && pool_k && pool_v && block_table, KVHP_ERR_INVALID,
                 "rmsnorm_qkv_rope_append: null pointer");
    KVHP_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && head_dim > 0 && head_dim % 16 == 0,
                 KVHP_ERR_INVALID, "rmsnorm_qkv_rope_append: head_dim %d must be a multiple of 16",
                 head_dim);
    KVHP_REQUIRE(max_pages > 0 && num_pages > 0, KVHP_ERR_INVALID,
                 "rmsnorm_qkv_rope_append: empty page pool");
    GemvArgs a = gemv_args(W_qkv, x, N, K);
    a.norm_w = static_cast<const f16*>(norm_w);
    a.eps = eps;
    a.y16 = static_cast<f16*>(q_out);
    a.Hq = num_q_heads;
    a.Hkv = num_kv_heads;
    a.D = head_dim;
    a.seq_len = seq_len;
    a.len_offset = len_offset;
    a.theta = rope_theta;
    a.pool_k = static_cast<f16*>(pool_k);
    a.pool_v = static_cast<f16*>(pool_v);
    a.bt = block_table;
    a.max_pages = max_pages;
    a.num_pages = num_pages;
    return launch_gemv<kEpiQKV, true>(a, static_cast<hipStream_t>(stream));
}

}  // namespace

extern "C" int kvhp_rmsnorm_qkv_rope_append(const void* W_qkv, const void* x, const void* norm_w,
                                            float eps, const int32_t* seq_len, float rope_theta,
                                            void* q_out, void* pool_k, void* pool_v,
                                            const int32_t* block_table, int max_pages,
                                            int num_pages, int num_q_heads, int num_kv_heads,
                                            int head_dim, int K, void* stream) {
    clear_error();
    return qkv_rope_append_impl(W_qkv, x, norm_w, eps, seq_len, 1, rope_theta, q_out, pool_k,
                                pool_v, block_table, max_pages, num_pages, num_q_heads,
                                num_kv_heads, head_dim, K, stream);
}

namespace kvhp {
int rmsnorm_qkv_rope_append_at(const void* W_qkv, const void* x, const void* norm_w, float eps,
                               const int32_t* position, float rope_theta, void* q_out,
                               void* pool_k, void* pool_v, const int32_t* block_table,
                               int max_pages, int num_pages, int num_q_heads, int num_kv_heads,
                               int head_dim, int K, hipStream_t stream) {
    return qkv_rope_append_impl(W_qkv, x, norm_w, eps, position, 0, rope_theta, q_out, pool_k,
                                pool_v, block_table, max_pages, num_pages, num_q_heads,
                                num_kv_heads, head_dim, K, stream);
}
}  // namespace kvhp

int residual_rows_impl(const void* W, const void* Wt, const void* x, const void* r, void* y,
                       int N, int K, int batch, void* workspace, size_t workspace_bytes,
                       hipStream_t s, const char* what, int x_tiles = 0, int y_tiles = 0) {
    if (N == 0 || batch == 0) return KVHP_OK;
    int rc = check_gemv(W ? W : Wt, x, N, K, what);
    if (rc) return rc;
    KVHP_REQUIRE(r && y, KVHP_ERR_INVALID, "%s: null residual/output", what);
    RowsArgs a{};
    a.W = static_cast<const f16*>(W);
    a.Wt = static_cast<const f16*>(Wt);
    a.x = static_cast<const f16*>(x);
    a.N = N;
    a.K = K;
    a.B = batch;
    a.resid = static_cast<const f16*>(r);
    a.y16 = static_cast<f16*>(y);
    a.ldy = N;
    a.x_tiles = x_tiles;
    a.y_tiles = y_tiles;
    const size_t need = ksplit_bytes(N, K, batch);
    if (need == 0 || workspace == nullptr) return launch_rows<kEpiResidual, false>(a, s, what);
    KVHP_REQUIRE(workspace_bytes >= need, KVHP_ERR_WORKSPACE,
                 "%s: workspace of %zu bytes, this call needs %zu", what, workspace_bytes, need);
    KVHP_REQUIRE(aligned16(W ? W : Wt) && aligned16(x) && aligned16(workspace),
                 KVHP_ERR_UNSUPPORTED, "%s: W, x and the workspace must be 16-byte aligned", what);
    return launch_ksplit_residual(a, static_cast<float*>(workspace), s, what);
}

extern "C" int kvhp_gemv_residual_rows(const void* W, const void* x, const void* r, void* y,
                                       int N, int K, int batch, void* stream) {
    clear_error();
    return residual_rows_impl(W, nullptr, x, r, y, N, K, batch, nullptr, 0,
                              static_cast<hipStream_t>(stream), "gemv_residual_rows");
}

extern "C" size_t kvhp_gemv_rows_workspace_bytes(int N, int K, int batch) {
    return ksplit_bytes(N, K, batch);
}

extern "C" int kvhp_gemv_residual_rows_ws(const void* W, const void* x, const void* r, void* y,
                                          int N, int K, int batch, void* workspace,
                                          size_t workspace_bytes, void* stream) {
    clear_error();
    return residual_rows_impl(W, nullptr, x, r, y, N, K, batch, workspace, workspace_bytes,
                              static_cast<hipStream_t>(stream), "gemv_residual_rows_ws");
}

extern "C" int kvhp_gemv_residual_rows_tiled(const void* W_tiled, const void* x, const void* r,
                                             void* y, int N, int K, int batch, void* workspace,
                                             size_t workspace_bytes, void* stream) {
    clear_error();
    KVHP_REQUIRE(W_tiled, KVHP_ERR_INVALID, "gemv_residual_rows_tiled: null weights");
    return residual_rows_impl(nullptr, W_tiled, x, r, y, N, K, batch, workspace,
                              workspace_bytes, static_cast<hipStream_t>(stream),
                              "gemv_residual_rows_tiled");
}

int rmsnorm_rows_impl(const void* W, const void* Wt, const void* x, const void* norm_w,
                      float eps, void* y16, float* y32, int N, int K, int batch, hipStream_t s,
                      const char* what, int act_tiles = 0) {
    if (N == 0 || batch == 0) return KVHP_OK;
    int rc = check_gemv(W ? W : Wt, x, N, K, what);
    if (rc) return rc;
    KVHP_REQUIRE(norm_w, KVHP_ERR_INVALID, "%s: null norm weight", what);
    KVHP_REQUIRE((y16 != nullptr) != (y32 != nullptr), KVHP_ERR_INVALID,
                 "%s: give exactly one of y16 / y32", what);
    RowsArgs a{};
    a.W = static_cast<const f16*>(W);
    a.Wt = static_cast<const f16*>(Wt);
    a.x = static_cast<const f16*>(x);
    a.norm_w = static_cast<const f16*>(norm_w);
    a.eps = eps;
    a.N = N;
    a.K = K;
    a.B = batch;
    a.y16 = static_cast<f16*>(y16);
    a.y32 = y32;
    a.ldy = N;
    a.x_tiles = act_tiles;
    a.y_tiles = y16 ? act_tiles : 0;
    return y32 ? launch_rows<kEpiF32, true>(a, s, what) : launch_rows<kEpiF16, true>(a, s, what);
}

extern "C" int kvhp_rmsnorm_gemv_rows(const void* W, const void* x, const void* norm_w, float eps,
                                      void* y16, float* y32, int N, int K, int batch,
                                      void* stream) {
    clear_error();
    return rmsnorm_rows_impl(W, nullptr, x, norm_w, eps, y16, y32, N, K, batch,
                             static_cast<hipStream_t>(stream), "rmsnorm_gemv_rows");
}

extern "C" int kvhp_rmsnorm_gemv_rows_tiled(const void* W_tiled, const void* x,
                                            const void* norm_w, float eps, void* y16, float* y32,
                                            int N, int K, int batch, void* stream) {
    clear_error();
    KVHP_REQUIRE(W_tiled, KVHP_ERR_INVALID, "rmsnorm_gemv_rows_tiled: null weights");
    return rmsnorm_rows_impl(nullptr, W_tiled, x, norm_w, eps, y16, y32, N, K, batch,
                             static_cast<hipStream_t>(stream), "rmsnorm_gemv_rows_tiled");
}

int swiglu_rows_impl(const void* W, const void* Wt, const void* x, const void* norm_w, float eps,
                     void* out, int N, int K, int batch, hipStream_t s, const char* what,
                     int act_tiles = 0) {
    if (N == 0 || batch == 0) return KVHP_OK;
    int rc = check_gemv(W ? W : Wt, x, N, K, what);
    if (rc) return rc;
    KVHP_REQUIRE(norm_w && out, KVHP_ERR_INVALID, "%s: null pointer", what);
    RowsArgs a{};
    a.W = static_cast<const f16*>(W);
    a.Wt = static_cast<const f16*>(Wt);
    a.x = static_cast<const f16*>(x);
    a.norm_w = static_cast<const f16*>(norm_w);
    a.eps = eps;
    a.N = N;
    a.K = K;
    a.B = batch;
    a.y16 = static_cast<f16*>(out);
    a.ldy = N;
    a.x_tiles = act_tiles;
    a.y_tiles = act_tiles;
    return launch_rows<kEpiSwiglu, true>(a, s, what);
}

extern "C" int kvhp_rmsnorm_gemv_swiglu_rows(const void* W_gate_up, const void* x,
                                             const void* norm_w, float eps, void* out, int N,
                                             int K, int batch, void* stream) {
    clear_error();
    return swiglu_rows_impl(W_gate_up, nullptr, x, norm_w, eps, out, N, K, batch,
                            static_cast<hipStream_t>(stream), "rmsnorm_gemv_swiglu_rows");
}

extern "C" int kvhp_rmsnorm_gemv_swiglu_rows_tiled(const void* W_tiled, const void* x,
                                                   const void* norm_w, float eps, void* out, int N,
                                                   int K, int batch, void* stream) {
    clear_error();
    KVHP_REQUIRE(W_tiled, KVHP_ERR_INVALID, "rmsnorm_gemv_swiglu_rows_tiled: null weights");
    return swiglu_rows_impl(nullptr, W_tiled, x, norm_w, eps, out, N, K, batch,
                            static_cast<hipStream_t>(stream), "rmsnorm_gemv_swiglu_rows_tiled");
}

int qkv_rows_impl(const void* W_qkv, const void* Wt, const void* x, const void* norm_w, float eps,
                  const int32_t* positions, float rope_theta, void* q_out, void* pool_k,
                  void* pool_v, const int32_t* block_tables, int max_pages, int num_pages,
                  int num_q_heads, int num_kv_heads, int head_dim, int K, int batch,
                  hipStream_t s, const char* what, int act_tiles = 0) {
    if (batch == 0) return KVHP_OK;
    const int N = (num_q_heads + 2 * num_kv_heads) * head_dim;
    int rc = check_gemv(W_qkv ? W_qkv : Wt, x, N, K, what);
    if (rc) return rc;
    KVHP_REQUIRE(norm_w && positions && q_out && pool_k && pool_v && block_tables,
                 KVHP_ERR_INVALID, "%s: null pointer", what);
    KVHP_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && head_dim > 0 && head_dim % 16 == 0,
                 KVHP_ERR_INVALID, "%s: head_dim %d must be a multiple of 16", what, head_dim);
    KVHP_REQUIRE(max_pages > 0 && num_pages > 0, KVHP_ERR_INVALID, "%s: empty page pool", what);
    RowsArgs a{};
    a.W = static_cast<const f16*>(W_qkv);
    a.Wt = static_cast<const f16*>(Wt);
    a.x = static_cast<const f16*>(x);
    a.norm_w = static_cast<const f16*>(norm_w);
    a.eps = eps;
    a.N = N;
    a.K = K;
    a.B = batch;
    a.y16 = static_cast<f16*>(q_out);
    a.ldy = num_q_heads * head_dim;
    a.Hq = num_q_heads;
    a.Hkv = num_kv_heads;
    a.D = head_dim;
    a.positions = positions;
    a.theta = rope_theta;
    a.pool_k = static_cast<f16*>(pool_k);
    a.pool_v = static_cast<f16*>(pool_v);
    a.bt = block_tables;
    a.max_pages = max_pages;
    a.num_pages = num_pages;
    a.x_tiles = act_tiles;
    return launch_rows<kEpiQKV, true>(a, s, what);
}

extern "C" int kvhp_rmsnorm_qkv_rope_append_rows(
    const void* W_qkv, const void* x, const void* norm_w, float eps, const int32_t* positions,
    float rope_theta, void* q_out, void* pool_k, void* pool_v, const int32_t* block_tables,
    int max_pages, int num_pages, int num_q_heads, int num_kv_heads, int head_dim, int K,
    int batch, void* stream) {
    clear_error();
    return qkv_rows_impl(W_qkv, nullptr, x, norm_w, eps, positions, rope_theta, q_out, pool_k,
                         pool_v, block_tables, max_pages, num_pages, num_q_heads, num_kv_heads,
                         head_dim, K, batch, static_cast<hipStream_t>(stream),
                         "rmsnorm_qkv_rope_append_rows");
}

extern "C" int kvhp_rmsnorm_qkv_rope_append_rows_tiled(
    const void* W_tiled, const void* x, const void* norm_w, float eps, const int32_t* positions,
    float rope_theta, void* q_out, void* pool_k, void* pool_v, const int32_t* block_tables,
    int max_pages, int num_pages, int num_q_heads, int num_kv_heads, int head_dim, int K,
    int batch, void* stream) {
    clear_error();
    KVHP_REQUIRE(W_tiled, KVHP_ERR_INVALID, "rmsnorm_qkv_rope_append_rows_tiled: null weights");
    return qkv_rows_impl(nullptr, W_tiled, x, norm_w, eps, positions, rope_theta, q_out, pool_k,
                         pool_v, block_tables, max_pages, num_pages, num_q_heads, num_kv_heads,
                         head_dim, K, batch, static_cast<hipStream_t>(stream),
                         "rmsnorm_qkv_rope_append_rows_tiled");
}

namespace kvhp {
namespace {
// Row-tiled activations need the batch's tile count and whole 32-column
// steps on both sides.
int check_act(int act_tiles, int batch, int K, int N, const char* what) {
    KVHP_REQUIRE(act_tiles == 0 || (act_tiles == act_tiles_for(batch) && K % 32 == 0 &&
                                    N % 32 == 0),
                 KVHP_ERR_INVALID, "%s: %d activation tiles for batch %d, K=%d N=%d", what,
                 act_tiles, batch, K, N);
    return KVHP_OK;
}
}  // namespace

int residual_rows_act(const void* Wt, const void* x, const void* r, void* y, int N, int K,
                      int batch, void* workspace, size_t workspace_bytes, int x_tiles,
                      int y_tiles, hipStream_t s) {
    if (int rc = check_act(x_tiles, batch, K, 32, "residual_rows_act")) return rc;
    if (int rc = check_act(y_tiles, batch, 32, N, "residual_rows_act")) return rc;
    return residual_rows_impl(nullptr, Wt, x, r, y, N, K, batch, workspace, workspace_bytes, s,
                              "residual_rows_act", x_tiles, y_tiles);
}

int rmsnorm_rows_act(const void* Wt, const void* x, const void* norm_w, float eps, void* y16,
                     float* y32, int N, int K, int batch, int act_tiles, hipStream_t s) {
    if (int rc = check_act(act_tiles, batch, K, y16 ? N : 32, "rmsnorm_rows_act")) return rc;
    return rmsnorm_rows_impl(nullptr, Wt, x, norm_w, eps, y16, y32, N, K, batch, s,
                             "rmsnorm_rows_act", act_tiles);
}

int swiglu_rows_act(const void* Wt, const void* x, const void* norm_w, float eps, void* out,
                    int N, int K, int batch, int act_tiles, hipStream_t s) {
    if (int rc = check_act(act_tiles, batch, K, N, "swiglu_rows_act")) return rc;
    return swiglu_rows_impl(nullptr, Wt, x, norm_w, eps, out, N, K, batch, s, "swiglu_rows_act",
                            act_tiles);
}

int qkv_rows_act(const void* Wt, const void* x, const void* norm_w, float eps,
                 const int32_t* positions, float rope_theta, void* q_out, void* pool_k,
                 void* pool_v, const int32_t* block_tables, int max_pages, int num_pages,
                 int num_q_heads, int num_kv_heads, int head_dim, int K, int batch, int act_tiles,
                 hipStream_t s) {
    if (int rc = check_act(act_tiles, batch, K, 32, "qkv_rows_act")) return rc;
    return qkv_rows_impl(nullptr, Wt, x, norm_w, eps, positions, rope_theta, q_out, pool_k,
                         pool_v, block_tables, max_pages, num_pages, num_q_heads, num_kv_heads,
                         head_dim, K, batch, s, "qkv_rows_act", act_tiles);
}

int embedding_act(const int32_t* token_ids, const void* table, void* out, int batch,
                  int64_t hidden, int64_t vocab, int act_tiles, hipStream_t s) {
    if (act_tiles == 0) return kvhp_embedding(token_ids, table, out, batch, hidden, vocab, s);
    if (batch <= 0) return KVHP_OK;
    KVHP_REQUIRE(token_ids && table && out && vocab > 0 && hidden > 0 && hidden % 32 == 0 &&
                     act_tiles == act_tiles_for(batch) && aligned16(table) && aligned16(out),
                 KVHP_ERR_INVALID, "embedding_act: bad arguments");
    hipLaunchKernelGGL(embedding_tiled_kernel, dim3(static_cast<unsigned>(batch)), dim3(256), 0, s,
                       token_ids, static_cast<const f16*>(table), static_cast<f16*>(out), hidden,
                       vocab, act_tiles);
    return check_launch("embedding_act");
}
}  // namespace kvhp

extern "C" size_t kvhp_rows_tiled_bytes(int kind, int N, int K, int num_q_heads,
                                        int num_kv_heads, int head_dim) {
    return static_cast<size_t>(rows_tiles(kind, N, K, num_q_heads, num_kv_heads, head_dim)) *
           32 * static_cast<size_t>(K > 0 ? K : 0);
}

extern "C" int kvhp_rows_tile_weights(int kind, const void* W, int N, int K, int num_q_heads,
                                      int num_kv_heads, int head_dim, void* W_tiled,
                                      void* stream) {
    clear_error();
    KVHP_REQUIRE(W && W_tiled, KVHP_ERR_INVALID, "rows_tile_weights: null pointer");
    KVHP_REQUIRE(aligned16(W) && aligned16(W_tiled), KVHP_ERR_UNSUPPORTED,
                 "rows_tile_weights: W and W_tiled must be 16-byte aligned");
    const int64_t tiles = rows_tiles(kind, N, K, num_q_heads, num_kv_heads, head_dim);
    KVHP_REQUIRE(tiles > 0, KVHP_ERR_UNSUPPORTED,
                 "rows_tile_weights: kind %d, N=%d, K=%d (heads %d/%d of %d) is not a shape the "
                 "batched projections take", kind, N, K, num_q_heads, num_kv_heads, head_dim);
    if (kind == KVHP_ROWS_QKV) N = (num_q_heads + 2 * num_kv_heads) * head_dim;
    const int64_t chunks = tiles * (K / 32) * kWave;
    hipLaunchKernelGGL(rows_tile_kernel, dim3(static_cast<unsigned>((chunks + 255) / 256)),
                       dim3(256), 0, static_cast<hipStream_t>(stream), static_cast<const f16*>(W),
                       static_cast<f16*>(W_tiled), kind, N, K, head_dim, chunks);
    return check_launch("rows_tile_weights");
}

extern "C" int kvhp_rmsnorm(const void* x, const void* weight, void* out, int64_t rows,
                            int64_t dim, float eps, void* stream) {
    clear_error();
    if (rows <= 0) return KVHP_OK;
    KVHP_REQUIRE(x && weight && out && dim > 0 && dim <= (1 << 24), KVHP_ERR_INVALID,
                 "rmsnorm: bad arguments");
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const f16*>(x),
                       static_cast<const f16*>(weight), static_cast<f16*>(out),
                       static_cast<int>(dim), eps);
    return check_launch("rmsnorm");
}

extern "C" int kvhp_apply_rope(void* q, void* k, int64_t seq_len, int64_t num_q_heads,
                               int64_t num_kv_heads, int64_t head_dim, int64_t start_pos,
                               float rope_theta, void* stream) {
    clear_error();
    if (seq_len <= 0) return KVHP_OK;
    KVHP_REQUIRE(q && k && head_dim > 0 && head_dim % 2 == 0 && num_q_heads > 0 &&
                     num_kv_heads > 0,
                 KVHP_ERR_INVALID, "apply_rope: bad arguments");
    const int64_t pairs = seq_len * (num_q_heads + num_kv_heads) * (head_dim / 2);
    hipLaunchKernelGGL(rope_kernel, dim3(grid_for(pairs, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<f16*>(q),
                       static_cast<f16*>(k), seq_len, static_cast<int>(num_q_heads),
                       static_cast<int>(num_kv_heads), static_cast<int>(head_dim),
                       static_cast<int>(start_pos), rope_theta);
    return check_launch("apply_rope");
}

extern "C" int kvhp_split_qkv_rope(const void* qkv, int64_t seq_len, int num_q_heads,
                                   int num_kv_heads, int head_dim, int64_t start_pos,
                                   float rope_theta, void* q, void* k, void* v, void* stream) {
    clear_error();
    if (seq_len <= 0) return KVHP_OK;
    KVHP_REQUIRE(qkv && q && k && v && head_dim > 0 && head_dim % 2 == 0 && num_q_heads > 0 &&
                     num_kv_heads > 0,
                 KVHP_ERR_INVALID, "split_qkv_rope: bad arguments");
    const int64_t pairs = seq_len * (num_q_heads + 2 * num_kv_heads) * (head_dim / 2);
    hipLaunchKernelGGL(split_qkv_rope_kernel, dim3(grid_for(pairs, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const f16*>(qkv), seq_len,
                       num_q_heads, num_kv_heads, head_dim, static_cast<int>(start_pos),
                       static_cast<const int32_t*>(nullptr), rope_theta, static_cast<f16*>(q),
                       static_cast<f16*>(k), static_cast<f16*>(v));
    return check_launch("split_qkv_rope");
}

extern "C" int kvhp_split_qkv_rope_rows(const void* qkv, int64_t rows, int num_q_heads,
                                        int num_kv_heads, int head_dim, const int32_t* positions,
                                        float rope_theta, void* q, void* k, void* v,
                                        void* stream) {
    clear_error();
    if (rows <= 0) return KVHP_OK;
    KVHP_REQUIRE(qkv && positions && q && k && v && head_dim > 0 && head_dim % 2 == 0 &&
                     num_q_heads > 0 && num_kv_heads > 0,
                 KVHP_ERR_INVALID, "split_qkv_rope_rows: bad arguments");
    const int64_t pairs = rows * (num_q_heads + 2 * num_kv_heads) * (head_dim / 2);
    hipLaunchKernelGGL(split_qkv_rope_kernel, dim3(grid_for(pairs, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const f16*>(qkv), rows,
                       num_q_heads, num_kv_heads, head_dim, 0, positions, rope_theta,
                       static_cast<f16*>(q), static_cast<f16*>(k), static_cast<f16*>(v));
    return check_launch("split_qkv_rope_rows");
}

extern "C" int kvhp_swiglu(const void* gate, const void* up, void* out, int64_t count,
                           void* stream) {
    clear_error();
    if (count <= 0) return KVHP_OK;
    KVHP_REQUIRE(gate && up && out, KVHP_ERR_INVALID, "swiglu: null pointer");
    hipLaunchKernelGGL(swiglu_kernel, dim3(grid_for(count, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const f16*>(gate),
                       static_cast<const f16*>(up), (int64_t)0, static_cast<f16*>(out),
                       (int64_t)1, count);
    return check_launch("swiglu");
}

extern "C" int kvhp_swiglu_rows(const void* gate_up, void* out, int64_t rows, int64_t n,
                                void* stream) {
    clear_error();
    if (rows <= 0 || n <= 0) return KVHP_OK;
    KVHP_REQUIRE(gate_up && out, KVHP_ERR_INVALID, "swiglu_rows: null pointer");
    const f16* g = static_cast<const f16*>(gate_up);
    hipLaunchKernelGGL(swiglu_kernel, dim3(grid_for(rows * n, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), g, g + n, 2 * n, static_cast<f16*>(out),
                       rows, n);
    return check_launch("swiglu_rows");
}

extern "C" int kvhp_embedding(const int32_t* token_ids, const void* table, void* out, int64_t n,
                              int64_t hidden, int64_t vocab, void* stream) {
    clear_error();
    if (n <= 0) return KVHP_OK;
    KVHP_REQUIRE(token_ids && table && out && hidden > 0 && vocab > 0, KVHP_ERR_INVALID,
                 "embedding: bad arguments");
    hipLaunchKernelGGL(embedding_kernel, dim3(static_cast<unsigned>(n)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), token_ids,
                       static_cast<const f16*>(table), static_cast<f16*>(out), n, hidden, vocab);
    return check_launch("embedding");
}

extern "C" int kvhp_argmax(const float* logits, int64_t n, int32_t* token, int32_t* seq_len,
                           int32_t* log, int32_t* log_count, void* stream) {
    clear_error();
    KVHP_REQUIRE(logits && token && n > 0 && n < (int64_t)1 << 31, KVHP_ERR_INVALID,
                 "argmax: bad arguments");
    KVHP_REQUIRE((log == nullptr) == (log_count == nullptr), KVHP_ERR_INVALID,
                 "argmax: log and log_count go together");
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream),
                       logits, n, token, seq_len, log, log_count, nullptr, int64_t{0}, nullptr);
    return check_launch("argmax");
}

extern "C" int kvhp_argmax_rows(const float* logits, int64_t rows, int64_t n, int32_t* tokens,
                                void* stream) {
    clear_error();
    if (rows <= 0) return KVHP_OK;
    KVHP_REQUIRE(logits && tokens && n > 0 && n < (int64_t)1 << 31 && rows <= 0x7fffffff,
                 KVHP_ERR_INVALID, "argmax_rows: bad arguments");
    hipLaunchKernelGGL(argmax_kernel, dim3(static_cast<unsigned>(rows)), dim3(1024), 0,
                       static_cast<hipStream_t>(stream), logits, n, tokens,
                       static_cast<int32_t*>(nullptr), static_cast<int32_t*>(nullptr),
                       static_cast<int32_t*>(nullptr), static_cast<const f16*>(nullptr),
                       int64_t{0}, static_cast<f16*>(nullptr));
    return check_launch("argmax_rows");
}

namespace kvhp {
int argmax_embed(const float* logits, int64_t n, int32_t* token, int32_t* seq_len, int32_t* log,
                 int32_t* log_count, const void* embed, int64_t hidden, void* x, hipStream_t s) {
    KVHP_REQUIRE(logits && token && embed && x && n > 0 && n < (int64_t)1 << 31 && hidden > 0,
                 KVHP_ERR_INVALID, "argmax_embed: bad arguments");
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, s, logits, n, token, seq_len, log,
                       log_count, static_cast<const f16*>(embed), hidden, static_cast<f16*>(x));
    return check_launch("argmax_embed");
}
}  // namespace kvhp

extern "C" int kvhp_randn_f16(void* out, int64_t count, uint64_t seed, uint64_t stream_id,
                              float std_dev, void* stream) {
    clear_error();
    if (count <= 0) return KVHP_OK;
    KVHP_REQUIRE(out, KVHP_ERR_INVALID, "randn: null output");
    hipLaunchKernelGGL(randn_kernel, dim3(grid_for(count, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<f16*>(out), count, seed,
                       stream_id, std_dev);
    return check_launch("randn_f16");
}

extern "C" int kvhp_fill_f16(void* out, int64_t count, float value, void* stream) {
    clear_error();
    if (count <= 0) return KVHP_OK;
    KVHP_REQUIRE(out, KVHP_ERR_INVALID, "fill: null output");
    hipLaunchKernelGGL(fill_kernel, dim3(grid_for(count, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<f16*>(out), count, value);
    return check_launch("fill_f16");
}
