/* theseus_gemm.h -- C ABI of the few-row GEMM in libtheseus_wkv7.so (gfx950).
 *
 * Y[M][N] = act(X[M][K] W[N][K]^T): bf16 in and out, float32 accumulation on the
 * matrix cores, for M <= THESEUS_GEMM_MAX_ROWS rows -- the projections and LoRAs of a
 * TimeMix serving step, where M is the number of lanes served at once and the product
 * streams the weight matrix (theseus/timemix.py:63-69: receptance, key, value, output
 * [C,C] and the LoRAs w1/w2, a1/a2, g1/g2 with the tanh and sigmoid between them).  The
 * reference runs these as torch matmuls (cuBLAS); a hipBLASLt GEMM at M = 64 spends most
 * of its time in a few output tiles without splitting K.  W is row-major [N][K]
 * (nn.Linear's [out][in]); a matrix stored [K][N] (the LoRAs) is passed transposed.
 * Results are deterministic (split-K partial tiles are summed in K order).
 */
#ifndef THESEUS_GEMM_H
#define THESEUS_GEMM_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hipStream_t;

#define THESEUS_GEMM_MAX_ROWS 128

enum theseus_gemm_act { THESEUS_GEMM_NONE = 0, THESEUS_GEMM_TANH = 1, THESEUS_GEMM_SIGMOID = 2 };

/* Workspace bytes theseus_gemm_rows needs for these sizes on the current device (0: none;
 * also 0 for sizes it refuses): the float32 partial tiles when K is split over several
 * workgroups (a second kernel sums them in K order).  Contents need not be initialised;
 * calls that may run at the same time must not share a workspace. */
size_t theseus_gemm_rows_workspace_size(int M, int N, int K);

/* Y = act(X W^T); x [M][K], w [N][K], y [M][N], all bf16 row-major and contiguous.  The
 * activation takes the product rounded to bf16, as a bf16 matmul followed by tanh /
 * sigmoid does under autocast.
 * Needs 1 <= M <= THESEUS_GEMM_MAX_ROWS, N a multiple of 16, K a multiple of 32
 * (THESEUS_WKV7_ERR_SHAPE otherwise), act a theseus_gemm_act (else THESEUS_WKV7_ERR_FLAGS).
 * Status codes are theseus_wkv7_status values; asynchronous on `stream`. */
int theseus_gemm_rows(int M, int N, int K, int act, const void* x, const void* w, void* y, void* workspace,
                      size_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* THESEUS_GEMM_H */
