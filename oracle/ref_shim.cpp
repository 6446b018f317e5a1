// ref_shim.cpp -- C entry points over the reference's own CPU ops.
//
// TEST INFRASTRUCTURE ONLY.  Compiled by oracle/Makefile together with the
// reference source src/cpu/ops.cpp where it lies (never copied) into
// oracle/_ref/libref_ops.so, which tests use to pin the oracle restatement
// bit-for-bit and bench.py may time as the CPU baseline.  The wrapped
// signatures are those of src/cpu/ops.h:21-123.
#include "src/cpu/ops.h"

extern "C" {

void ref_causal_gqa(const float* q, const float* k, const float* v, float* out,
                    int64_t S, int64_t Hq, int64_t Hkv, int64_t D) {
    engine::cpu::causal_gqa(q, k, v, out, S, Hq, Hkv, D);
}

void ref_rmsnorm(const float* x, const float* w, float* out, int64_t rows,
                 int64_t dim, float eps) {
    engine::cpu::rmsnorm(x, w, out, rows, dim, eps);
}

void ref_matmul_transB_blocked(const float* A, const float* B, float* C,
                               int64_t M, int64_t K, int64_t N) {
    engine::cpu::matmul_transB_blocked(A, B, C, M, K, N);
}

void ref_apply_rope(float* q, float* k, int64_t S, int64_t Hq, int64_t Hkv,
                    int64_t D, int64_t start_pos, float theta) {
    engine::cpu::apply_rope(q, k, S, Hq, Hkv, D, start_pos, theta);
}

void ref_swiglu(const float* gate, const float* up, float* out, int64_t n) {
    engine::cpu::swiglu(gate, up, out, n);
}

}  // extern "C"
