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
#define THESEUS_GEMM_MAX_GROUP 8

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

/* One product of a group: y [M][N] = act(x [M][K] w [N][K]^T), as theseus_gemm_rows. */
typedef struct theseus_gemm_problem {
    int N, K, act;
    const void* x;
    const void* w;
    void* y;
} theseus_gemm_problem;

/* Workspace bytes of theseus_gemm_rows_group (0: none, or sizes it refuses). */
size_t theseus_gemm_rows_group_workspace_size(int M, int count, const theseus_gemm_problem* probs);

/* 1 <= count <= THESEUS_GEMM_MAX_GROUP independent products with the same M in one launch
 * (a serving step's r, k, v projections and LoRA first halves, which all read the step's
 * token mixes; then the LoRA second halves): each product takes a share of the CUs in
 * proportion to its weight bytes, so the 5120-wide projections run one workgroup per
 * column tile with no K split and no second kernel, where a lone projection splits K to
 * fill the chip.  Results equal theseus_gemm_rows' for each product up to the order of
 * the float32 sums.  Errors as theseus_gemm_rows for any product; probs is read on the
 * host during the call only. */
int theseus_gemm_rows_group(int M, int count, const theseus_gemm_problem* probs, void* workspace,
                            size_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* THESEUS_GEMM_H */
