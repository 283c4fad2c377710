/*
 * spanqr.h -- C ABI of the MI355X (gfx950) implementation of spanqr's orth(X).
 *
 * orth(X) returns Q with orthonormal columns and span(Q) = span(X) for a tall fp32 matrix X [K, r] (K >= r), using
 * the robust shifted Cholesky-QR of the reference ("kcholf"): power-of-2 scale on load, seeded dust in the first
 * solve, three passes of {Gram, shift, pivot-clamped Cholesky, triangular solve}, two Newton-Schulz polish steps.
 *
 * Conventions
 *   - Matrices are row-major fp32 in device memory; X and Q need 16-byte alignment and a leading dimension that is a
 *     multiple of 4 and below 2^24 (the contiguous [K, r] case always qualifies). X is never written.
 *   - r must be a multiple of 32 with 32 <= r <= 1024 (kcholf at full width), or a multiple of 256 with
 *     512 < r <= 4096 (the column-blocked path: block Gram-Schmidt over 256-column blocks, as the reference's orth
 *     does above 512 columns; spanqr_plan_create picks it for those r); K >= r.
 *   - Every entry point that takes a stream only enqueues work on it: no host synchronisation, no allocation, so a
 *     call can be captured into a hipGraph. Plan creation allocates and synchronises.
 *   - Return value 0 means success; a negative value is an error whose message spanqr_last_error() returns (per
 *     thread). Nothing is thrown across the ABI.
 *   - A plan owns its workspace (dust, Gram partials, Cholesky factors, solve buffers, grid-barrier counters). Calls on
 *     one plan must not overlap in time (same stream, or externally ordered); use one plan per concurrent stream.
 */
#ifndef SPANQR_H
#define SPANQR_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct spanqr_plan spanqr_plan;

/* Most matrices one spanqr_orth_batched_f32 call takes. */
#define SPANQR_MAX_BATCH 32

/* Widest X a plan takes: above 512 columns (a multiple of 256) the plan is column-blocked (see spanqr_plan_create). */
#define SPANQR_MAX_R 4096
/* Widest X kcholf runs on at full width (candidates/kcholqr.py:92-112 with chol.cu's Cholesky, n <= ~1024). */
#define SPANQR_KCHOLF_MAX_R 1024

enum {
    SPANQR_OK = 0,
    SPANQR_EINVAL = -1,     /* bad argument (shape, alignment, null pointer) */
    SPANQR_EHIP = -2,       /* a HIP runtime call failed */
    SPANQR_ENOMEM = -3,     /* workspace allocation failed */
};

/* Plan queries for spanqr_plan_query. */
enum {
    SPANQR_Q_K = 0,
    SPANQR_Q_R = 1,
    SPANQR_Q_SPLITS = 2,         /* Gram row splits S */
    SPANQR_Q_SPLIT_ROWS = 3,     /* rows per split KS (a multiple of 32) */
    SPANQR_Q_CHOL_GRID = 4,      /* workgroups of one matrix's Cholesky (max(1, r/32 - 3)) */
    SPANQR_Q_WORKSPACE_MB = 5,   /* workspace size, MiB (rounded up) */
    SPANQR_Q_DEVICE = 6,
    SPANQR_Q_BATCH = 7,          /* matrices per call the plan holds workspace for */
    SPANQR_Q_CHOL_BATCH = 8,     /* matrices per Cholesky launch (all their workgroups fit on the device at once) */
    SPANQR_Q_BLOCKS = 9,         /* column blocks of a column-blocked plan (r > 512, or spanqr_plan_create_borth); 0
                                    otherwise */
    SPANQR_Q_SOLVE_ROWS = 10,    /* rows per solve workgroup when the solve runs in the Cholesky's launch; 0 when
                                    they are separate launches */
    SPANQR_Q_BLOCK_WIDTH = 11,   /* columns per block of a column-blocked plan; 0 otherwise */
    SPANQR_Q_NORM_PARTIALS = 12, /* fp64 partials of ||G||_F^2 per matrix that the Gram writes (spanqr_norm_partials) */
};

/* Create a plan for X [K, r] on HIP device `device` (allocates the workspace and uploads the dust matrix), with
 * orth's dispatch (orth.py:13-20). Replaces the per-call allocations and module-level caches of the reference: the
 * dust cache _Z (candidates/kcholqr.py:26, :83-89), chol32's G clone / L / Li / barrier (candidates/kchol.py:12-18,
 * :40-42) and the Gram partials (candidates/tri.py:371). For r > 512 a multiple of 256 (up to SPANQR_MAX_R) the plan
 * is column-blocked (borth, candidates/kbig.py:69-95, called from orth.py:18-19 with 256-column blocks): it holds the
 * plan of one 256-column block, the K x r dust whose column slices the blocks use (_ZB, kbig.py:76-83) and the
 * projection's buffers; such a plan runs spanqr_orth_f32 only (the stage, profiling and batched entry points return
 * SPANQR_EINVAL for it). Any other r a multiple of 32 up to SPANQR_KCHOLF_MAX_R runs kcholf at full width
 * (orth.py:20), as spanqr_plan_create_batched with batch = 1. */
int spanqr_plan_create(int K, int r, int device, spanqr_plan** out);

/* Plan for kcholf at full width (candidates/kcholqr.py:92-112) on up to `batch` (1..SPANQR_MAX_BATCH) matrices
 * [K, r] per call (spanqr_orth_batched_f32): r a multiple of 32 in [32, SPANQR_KCHOLF_MAX_R], one workspace per
 * matrix, one shared dust matrix. Differs from spanqr_plan_create only at r = 768 and 1024, where this is the
 * full-width kcholf of kcholqr_f and spanqr_plan_create the column-blocked orth. */
int spanqr_plan_create_batched(int K, int r, int batch, int device, spanqr_plan** out);

/* Column-blocked plan for borth(X, b, reorth) (candidates/kbig.py:69-95, whose parameters these are): block
 * Gram-Schmidt over b-column blocks, each block projected twice against the finished ones and orthonormalised by
 * kcholf at width b with its column slice of the K x r dust; with reorth != 0 projected and orthonormalised once more
 * (kbig.py:91-92). b a multiple of 32 in [32, 1024], r > b a multiple of b up to 4096, K >= r (the reference runs
 * kcholf at full width when r <= b or r % b != 0: the caller's choice, kbig.py:77-78). spanqr_orth_f32 on the plan
 * runs it (eps, alpha, tau, ns apply to every block's kcholf); spanqr_plan_create for r > 512 is b = 256 with reorth,
 * the call orth.py:19 makes. */
int spanqr_plan_create_borth(int K, int r, int b, int reorth, int device, spanqr_plan** out);
void spanqr_plan_destroy(spanqr_plan* plan);
long spanqr_plan_query(const spanqr_plan* plan, int what);

/* Q = orth(X) with the reference's keyword arguments (defaults eps 5e-7, alpha 1e-7, tau 1e-8, ns 2).
 * Replaces orth (orth.py:13-20): on a kcholf plan kcholqr_f (candidates/kcholqr.py:92-112); on a column-blocked plan
 * borth(X, 256) (candidates/kbig.py:69-95): per 256-column block, W = s X_blk (s of the whole X), twice
 * W -= P (P^T W) against the finished columns P, the kcholf recipe on W with the block's dust slice (kbig.py:50-63),
 * then once more W -= P (P^T W) and the recipe again. stream: a hipStream_t (torch.cuda.current_stream().cuda_stream
 * on ROCm), 0 for the null stream. */
int spanqr_orth_f32(spanqr_plan* plan, const float* X, long ldx, float* Q, long ldq, float eps, float alpha,
                    float tau, int ns, void* stream);

/* Q[i] = orth(X[i]) for the n <= batch matrices of one shape group: X and Q are host arrays of n device pointers
 * (read at the call, so a captured graph keeps them), all with leading dimensions ldx and ldq. Each kernel of the
 * call runs once for all n matrices (blockIdx.z is the matrix); the Cholesky runs in launches of at most
 * SPANQR_Q_CHOL_BATCH matrices. Q[i] is bit-identical to spanqr_orth_f32 on X[i] alone. No counterpart in the
 * reference, whose caller orthonormalises layer by layer (qrbench/methods.py:47-50) and names batching as the next
 * step (README.md:91-92, METHODS.md:93, :102-103). */
int spanqr_orth_batched_f32(spanqr_plan* plan, int n, const float* const* X, long ldx, float* const* Q, long ldq,
                            float eps, float alpha, float tau, int ns, void* stream);

/* Allocation-free form of spanqr_orth_f32. No counterpart in the reference: for callers that cannot allocate device
 * memory (code under hipGraph capture, tight serving loops, harnesses that forbid hipMalloc). Q = orth(X) for
 * X [K, r] on the current device, bit-identical to spanqr_orth_f32 on a plan for (K, r), but without a plan: the
 * workspace lives in a fixed 64 MiB device array of the library (each GPU the library runs on holds its own copy
 * until the process ends), and nothing is allocated or synchronised. Limits: r a multiple of 32 in [32, 512] (no
 * column-blocked path), K >= r, and the workspace of (K, r) within 64 MiB (17408 x 256 fits; 32768 x 512 does
 * not): larger shapes return SPANQR_EINVAL. The dust is generated on the device and kept with a shape tag, so a call
 * after one of another shape regenerates it (a few extra kernels). Every call on one GPU shares the array, which
 * keeps the last call's contents: calls that overlap in time on one GPU (other streams or threads) race, and the
 * caller must order them. */
int spanqr_orth_f32_noalloc(int K, int r, const float* X, long ldx, float* Q, long ldq, float eps, float alpha,
                            float tau, int ns, void* stream);

/* Profiling form of spanqr_orth_f32: the same kernels on the same stream with a HIP event after each, then waits
 * for the stream (host synchronisation: not for the hot path). ms[i] receives the time of kernel i in launch order
 * (amax; per pass gram, reduce, chol, trsm; per polish step gram, reduce, apply); *n_out their number.
 * No counterpart in the reference (its bench times whole calls, qrbench/bench.py:28-53). */
int spanqr_profile_orth(spanqr_plan* plan, const float* X, long ldx, float* Q, long ldq, float eps, float alpha,
                        float tau, int ns, void* stream, float* ms, int max_n, int* n_out);

/* Profiling form of the Cholesky stage (spanqr_stage_chol with npart): runs an instrumented copy of the kernel whose
 * workgroup 0 stamps the device wall clock, copies 24 r/32 + 2 stamps to host memory and waits for the stream: [0]
 * kernel start; for each 32-column diagonal step j (nb = r/32 steps), [1 + 4j] step start, [2 + 4j] step end (the
 * whole workgroup), [3 + 4j] the look-ahead's wavefront done, [4 + 4j] the tile factor's wavefront done; [1 + 4 nb]
 * end; [2 + 4 nb + j] tile row j+2's wavefronts done; [2 + 5 nb + j] the publishing wavefront done; [2 + 6 nb + j]
 * the hand-over of row j+2 seen; [2 + 7 nb + j] row j+2 fetched; [2 + 8 nb + j] its panel L(j+2, j-1) formed;
 * [2 + 9 nb + j] the second of row j+2's wavefronts done; for the owner of tile row i (its last part, at the
 * block before it hands the row over), [2 + 10 nb + 6i + s]: s = 0 the block's flags seen, 1 operands loaded,
 * 2 panels formed, 3 row handed over, 4 row updated, 5 hand-over stores done; for the last tile row's last part at
 * block j, [2 + 16 nb + 8j + s]: s = 0 flags seen, 1 operands loaded, 2 panels formed, 3 block done, 4 the next
 * block's tile published; zero where a step has no such work. *tick_ns: nanoseconds per wall-clock tick. The reference keeps similar
 * stamps behind a debug define (candidates/cuk/chol.cu:17-23). */
int spanqr_profile_chol(spanqr_plan* plan, const float* G, const double* npart, float alpha, float tau,
                        unsigned long long* stamps_out, double* tick_ns, void* stream);

/* Kernels for spanqr_profile_kernel (the pass-1 forms read the power-of-2 scale and, for the solve, the dust). */
enum {
    SPANQR_K_AMAX = 0,
    SPANQR_K_GRAM_PASS1 = 1,     /* Kahan Gram, scaled on load */
    SPANQR_K_GRAM = 2,           /* plain Gram */
    SPANQR_K_REDUCE = 3,         /* fp64 split reduction + norm partials */
    SPANQR_K_CHOL = 4,           /* flag-synchronised clamped Cholesky */
    SPANQR_K_TRSM_PASS1 = 5,     /* solve with the fused s * x + eps * z operand */
    SPANQR_K_TRSM = 6,           /* solve */
    SPANQR_K_NS_APPLY = 7,       /* Newton-Schulz correction Y + Y D */
    SPANQR_K_CHOL_SOLVE_PASS1 = 8,   /* the Cholesky with the pass-1 solve in one launch (plans with SOLVE_ROWS > 0) */
    SPANQR_K_CHOL_SOLVE = 9,         /* the Cholesky with the solve in one launch */
};

/* Average duration of one kernel of the call: `reps` back-to-back launches on the plan's own workspace, between two
 * HIP events on `stream`, after one untimed launch (the Cholesky-with-solve launches: each between its own pair of
 * events, after a small kernel that resets its column counters); waits for the stream. For timing only: it leaves the workspace
 * in an unspecified state (the next spanqr_orth_f32 rebuilds what it needs). No counterpart in the reference. */
int spanqr_profile_kernel(spanqr_plan* plan, int which, int reps, float* avg_ms, void* stream);

/* Message of the last failed call on this thread ("" if none). */
const char* spanqr_last_error(void);

/* Host-side dust generator (no GPU needed): Z [K, r] row-major, unit columns, the matrix every plan uploads.
 * Replaces _zdust (candidates/kcholqr.py:83-89), whose torch CUDA Philox stream is NVIDIA-specific; this generator
 * is seeded with the same 20261018 and defined in the source (splitmix64 counter hash, Irwin-Hall(12) normals). */
int spanqr_dust_host(int K, int r, float* Z);

/* Host-side split policy (no GPU needed): rows per Gram split KS (a multiple of 32) for X [K, r]; the Gram runs
 * ceil(K / KS) splits. Same rule as gram_f (candidates/tri.py:364-367) with a fixed target of 512 workgroups in place
 * of 3 x the device's SM count, so the summation order, and with it every bit of Q, is the same on every device.
 * Returns SPANQR_EINVAL for a shape the plan would reject. */
int spanqr_split_rows(int K, int r);

/* Host-side (no GPU needed): the number of fp64 ||G||_F^2 partials the Gram of X [K, r] writes, which also tells its
 * form: short X with many tiles (K <= 1024, r >= 448) runs the Gram in one launch over upper 32 x 32 tiles, two row splits of
 * spanqr_split_rows(K, r) rows summed in fp64 inside each tile's workgroup, one partial per tile (r/32 (r/32 + 1) / 2);
 * other X runs the split Gram over upper 64 x 64 tiles and a reduction launch, 16 partials per tile. Both give every
 * element of G the same arithmetic for the same split; the partials' grouping differs, and with it the bits of ||G||_F
 * (the reference computes it with torch.linalg.matrix_norm, candidates/kcholqr.py:107; the oracle restates both forms).
 * No counterpart in the reference. Returns SPANQR_EINVAL for a shape the plan would reject. */
int spanqr_norm_partials(int K, int r);

/* ---- stage entry points: one stage of the call on device buffers, for checking each kernel ---- */

/* max|x| partials of X into the plan (the scale the pass-1 kernels derive from them is written to scal[0] by
 * the pass-1 solve). Replaces torch.linalg.vector_norm(X, inf) + _pow2_scale (candidates/kcholqr.py:29-30, :102). */
int spanqr_stage_amax(spanqr_plan* plan, const float* X, long ldx, void* stream);

/* G = A^T A [r, r] (Kahan within a split when kahan != 0, fp64 across splits; scaled on load by the plan's
 * current power-of-2 scale when use_scale != 0) and the fp64 partials of ||G||_F^2 (16 per upper 64x64 tile, or
 * NULL). Replaces gram_f / gram_split (candidates/tri.py:324-375, :255-297) and Y.T @ Y (kcholqr.py:106). */
int spanqr_stage_gram(spanqr_plan* plan, const float* A, long lda, int use_scale, int kahan, float* G,
                      double* npart, void* stream);

/* Clamped Cholesky of G + fp32(alpha ||G||_F) I with pivot floor fp32(tau ||G||_F) + 1e-30, ||G||_F from npart;
 * with npart NULL, of G itself with the absolute pivot floor tau (alpha ignored), which is chol32's contract:
 * L [r, r] lower (upper triangle of the diagonal tiles zero; upper tiles untouched) and Li [r, 32] the inverses of
 * the 32x32 diagonal tiles; scal (3 floats, may be NULL) receives {nrm, tau, reserved}. G is not modified.
 * Replaces the shift at candidates/kcholqr.py:107-109 and chol32 (candidates/kchol.py:35-44) -> chol_f32
 * (candidates/cuk/chol.cu:273-276). */
int spanqr_stage_chol(spanqr_plan* plan, const float* G, const double* npart, float alpha, float tau, float* L,
                      float* Li, float* scal, void* stream);

/* Y = A L^-T (blocked, 32-wide diagonal blocks through Li). With pass1 != 0 the operand is fmaf(eps, Z, s * A)
 * with the plan's dust Z and scale s (spanqr_stage_amax first). Replaces trsm_f (candidates/tri.py:378-412). */
int spanqr_stage_trsm(spanqr_plan* plan, const float* A, long lda, int pass1, float eps, const float* L,
                      const float* Li, float* Y, long ldy, void* stream);

/* One Newton-Schulz polish step Yout = Y + Y fp32(I - G) / 2 with G = Y^T Y (Kahan Gram when kahan != 0).
 * Replaces one iteration of _ns_mm (candidates/kcholqr.py:16-23). */
int spanqr_stage_ns(spanqr_plan* plan, const float* Y, long ldy, int kahan, float* Yout, long ldo, void* stream);

/* Copy the plan's dust matrix (device) and the scalars of the last call's first matrix {s, nrm0, tau0, nrm1, tau1,
 * nrm2, tau2, wait error} (device, 8 floats; the last is nonzero if a bounded wait of that call's Cholesky gave up:
 * every call clears it first, and such a call's Q is NaN). */
int spanqr_plan_copy_dust(spanqr_plan* plan, float* Z, void* stream);
int spanqr_plan_copy_scalars(spanqr_plan* plan, float* scal8, void* stream);

/* Host-visible outcome of the last call enqueued on the plan (spanqr_orth_f32, spanqr_orth_batched_f32 with its n
 * matrices, spanqr_chol32): synchronises the stream, then returns SPANQR_OK, or SPANQR_EHIP naming the first matrix
 * whose Cholesky gave up a bounded wait (its Q is NaN). The reference launches its Cholesky cooperatively
 * (candidates/kchol.py:43, cudak.py:95-106), so a launch that cannot be co-scheduled fails there with a CUresult;
 * here the launch is an ordinary one whose flag waits need every workgroup resident, and a wait that gives up after
 * ~1 s of polling (another kernel holding the CUs) turns that matrix's Q into NaN without a host synchronisation.
 * This call is the opt-in check for it (not for the hot path: it synchronises). */
int spanqr_plan_status(spanqr_plan* plan, void* stream);

/* chol32(G, tau) (candidates/kchol.py:35-44 -> chol_f32, candidates/cuk/chol.cu:273-276): the clamped Cholesky of
 * G [n, n] fp32 (lower triangle read, row stride ldg >= n; not modified) with the absolute pivot floor *tau (a device
 * pointer to one float, as the reference passes it: no host synchronisation) and no shift. Writes L [n, n] (row
 * stride ldl >= n; zeros above the diagonal) and Li [n, 32] (the inverses of L's 32 x 32 diagonal tiles). plan: a
 * kcholf plan with r = n (spanqr_plan_create_batched(K, n, 1, ...) for any K >= n; its workspace holds the
 * factorisation's scratch and flags, so calls on one plan must not overlap). spanqr_plan_status reports a wait that
 * gave up (L and Li are then unspecified). */
int spanqr_chol32(spanqr_plan* plan, const float* G, long ldg, const float* tau, float* L, long ldl, float* Li,
                  void* stream);

/* Testing only (no counterpart in the reference): polls one bounded wait of the Cholesky makes before it gives up
 * (default 2^20, about a second). Lowered to 0, a wait gives up unless its flag is already set, so the tests can
 * exercise the failure path with every kernel still ending normally: the wait-error word is set and the call's Q
 * comes out NaN. Applies to launches made after the call (a captured graph keeps the value it was captured with).
 * Not thread-safe with concurrent launches; restore the default (1048576) afterwards. */
int spanqr_debug_spin_limit(unsigned polls);

/* ---- fp64 clamped Cholesky (kchol.chol64, candidates/kchol.py:47-57 -> chol_f64, candidates/cuk/chol.cu:278-281) ----
 * A plan holds the flag words of one n x n factorisation (n a multiple of 32 up to 1024); one plan per concurrent
 * stream. spanqr_chol64: G [n, n] fp64 (lower tiles read, row stride ldg, even), tau a device pointer to the fp64
 * pivot floor (as the reference passes it, no host synchronisation); writes L [n, n] fp64 (zeros above the
 * diagonal), Li [n, 32] fp64 (inverses of the 32x32 diagonal tiles) and their fp32 copies Lf [n, n], Lif [n, 32].
 * Pivots below tau (or NaN) are clamped to tau. spanqr_chol64_status synchronises the stream and reports a wait
 * that gave up (which can only happen if not every workgroup of the launch was resident). */
typedef struct spanqr_chol64_plan spanqr_chol64_plan;
int spanqr_chol64_plan_create(int n, int device, spanqr_chol64_plan** out);
void spanqr_chol64_plan_destroy(spanqr_chol64_plan* plan);
int spanqr_chol64(spanqr_chol64_plan* plan, const double* G, long ldg, const double* tau, double* L, double* Li,
                  float* Lf, float* Lif, void* stream);
int spanqr_chol64_status(spanqr_chol64_plan* plan, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SPANQR_H */
