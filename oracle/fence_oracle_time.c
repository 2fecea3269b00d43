/*
 * fence_oracle_time.c -- CPU-baseline timing over the scalar oracle.
 *
 * TEST INFRASTRUCTURE ONLY: the cpu_baseline leg of bench.py calls these to
 * time the oracle on the host.  The oracle calls run on caller-owned buffers
 * between two CLOCK_MONOTONIC reads, so the interval holds no allocation, no
 * copy and no Python.
 */
#define _POSIX_C_SOURCE 199309L
#include <time.h>

#include "fence_oracle.h"

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

void fo_time_elementwise_stage(double secs[3], int reps, float* scores, int64_t heads, int sq,
                               int sk, float* act, const float* gate, const float* up, int64_t n,
                               float* q, float* k, int64_t tokens, int n_q_heads, int n_kv_heads,
                               int head_dim, const int32_t* positions, float freq_base, int style) {
    secs[0] = secs[1] = secs[2] = 0.0;
    for (int r = 0; r < reps; ++r) {
        const double t0 = now_s();
        fo_softmax_causal(scores, heads, sq, sk);
        const double t1 = now_s();
        fo_silu_elementwise_mul(act, gate, up, n);
        const double t2 = now_s();
        fo_rope_rows(q, k, tokens, n_q_heads, n_kv_heads, head_dim, positions, 0, freq_base, style);
        const double t3 = now_s();
        secs[0] += t1 - t0;
        secs[1] += t2 - t1;
        secs[2] += t3 - t2;
    }
}
