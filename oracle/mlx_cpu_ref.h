/*
 * mlx_cpu_ref.h — CPU oracle for mlx-hip parity tests (TEST INFRASTRUCTURE).
 *
 * A plain-C restatement of the reference's CPU backend, CpuRefBackend
 * (crates/mlx-core/src/cpu_kernels.rs), and of its test-data generator
 * gen_data (crates/mlx-parity/src/lib.rs:22-39). Only the test suite, the
 * smoke check and the benchmark's CPU-baseline leg use it, always as the
 * checker; the mlx-hip library never links or calls it.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no -ffast-math), so that
 * every f32 operation rounds exactly as Rust's strict f32 arithmetic does and
 * expf/logf/tanhf/sqrtf/powf/sinf/cosf are the same glibc routines Rust's std
 * calls on x86-64 Linux.
 *
 * Parity pinning status per function is listed in mlx_cpu_ref.c's header.
 */
#ifndef MLX_CPU_REF_H
#define MLX_CPU_REF_H

#include <stddef.h>
#include <stdint.h>

#include "../include/mlxhip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* CpuRefBackend::eval_node (cpu_kernels.rs:13-102). On success (*out, *out_len)
 * hold a malloc'd result the caller releases with oracle_free. Returns an
 * mlxhip_status_t; the message is available from oracle_last_error(). */
int oracle_eval_node(const mlxhip_op_t* op, const mlxhip_input_t* inputs, size_t n_inputs,
                     const mlxhip_meta_t* out_meta, float** out, size_t* out_len);
void oracle_free(float* p);
const char* oracle_last_error(void);

/* gen_data / gen_positive_data (crates/mlx-parity/src/lib.rs:22-39). */
void oracle_gen_data(float* out, size_t n, uint64_t seed);
void oracle_gen_positive_data(float* out, size_t n, uint64_t seed);

/* Direct kernels used by the CPU baseline timing (same code the dispatch uses). */
void oracle_matmul(const float* a, const float* b, float* c, size_t m, size_t k, size_t n);
/* Rows [row0, row0+nrows) of the same product (for bounded CPU samples). */
void oracle_matmul_rows(const float* a, const float* b, float* c, size_t m, size_t k,
                        size_t n, size_t row0, size_t nrows);
void oracle_softmax_lastdim(const float* x, float* y, size_t rows, size_t cols);
void oracle_layer_norm(const float* x, float* y, size_t rows, size_t cols, float eps);
void oracle_rms_norm(const float* x, float* y, size_t rows, size_t cols, float eps);

#ifdef __cplusplus
}
#endif

#endif
