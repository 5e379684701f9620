/*
 * fp64emu.h -- C ABI of the MI355X-native RARE emulated-FP64 GEMM.
 *
 * C = A @ B in float64 is recovered from INT8 products modulo up to 20
 * pairwise-coprime moduli (one CDNA4 INT8-MFMA GEMM each), a first-order
 * quantization correction (hi7 x q7 cross GEMMs) and balanced-Garner
 * reconstruction.  Every entry point enqueues asynchronously on `stream`
 * and allocates nothing: the caller passes a 256-byte aligned device
 * workspace of at least fp64emu_workspace_size() bytes (hipMalloc and the
 * torch caching allocator, which the binding uses and which keeps the call
 * graph-capturable, both align that far).  All pointers
 * are device pointers unless the parameter says "host".
 *
 * Return value: 0 on success, nonzero on error; fp64emu_last_error() then
 * holds the message (thread-local).  The messages of argument errors are
 * the reference's TORCH_CHECK texts.
 *
 * Reference interface each entry point replaces (paths relative to the
 * upstream fp64-emu checkout):
 *   torch-ext/torch_binding.cpp:7-12   op schemas
 *   torch-ext/torch_binding.h:5-21     C++ signatures
 *   fp64_emu_cuda/fp64_emu.cu:956      fp64_emu_maxp
 *   fp64_emu_cuda/fp64_emu.cu:1583     fp64_emu_mm
 *   fp64_emu_cuda/fp64_emu.cu:1613     fp64_emu_mm_nt
 *   fp64_emu_cuda/fp64_emu.cu:1637     fp64_emu_bmm
 *   fp64_emu_cuda/fp64_emu.cu:1665     fp64_emu_bmm_nt
 *   fp64_emu_cuda/fp64_emu.cu:1688     fp64_emu_mm_timed
 * The reference's `Tensor primes_cpu, Tensor inv_cpu, Tensor mu_cpu` become
 * host pointers plus `nprimes`; like the reference (fp64_emu.cu:1137-1140)
 * the library derives its own tables from `primes` and ignores `inv`/`mu`,
 * which may be NULL.
 */
#ifndef FP64EMU_H
#define FP64EMU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t / hipEvent_t, kept opaque so this header needs no HIP include. */
typedef struct ihipStream_t* fp64emu_stream_t;
typedef struct ihipEvent_t* fp64emu_event_t;

#define FP64EMU_MAXP 20

enum {
  FP64EMU_OK = 0,
  FP64EMU_EINVAL = 1,     /* argument check failed (reference TORCH_CHECK) */
  FP64EMU_EWORKSPACE = 2, /* workspace missing or too small */
  FP64EMU_EHIP = 3        /* HIP runtime error (launch, event) */
};

/* fp64_emu_cuda/fp64_emu.cu:956 -- the largest modulus count (20). */
int fp64emu_maxp(void);

/* Message of the last failed call on this thread ("" if none). */
const char* fp64emu_last_error(void);

/* Device workspace bytes needed by one call with these shapes (per batch
 * member M, N, K).  Replaces the per-call torch::empty/zeros scratch of
 * run_crt (fp64_emu_cuda/fp64_emu.cu:1148-1151, 1255-1256, 1344-1345). */
size_t fp64emu_workspace_size(int64_t batch, int64_t M, int64_t N, int64_t K,
                              int nprimes, int use_corr);

/* The smallest workspace a call accepts.  With less than
 * fp64emu_workspace_size() bytes, a call of fp64emu_mm, fp64emu_mm_nt or
 * fp64emu_mm_nt_noalloc with K <= 131071 runs the rows of A in chunks of
 * 256-row multiples against one extraction of B (the fewest chunks that
 * fit), so products too large for the full workspace still run.  Other
 * calls (batched, K-segmented, and the phase-timed fp64emu_mm_timed and
 * fp64emu_mm_nt_events, whose events bracket whole phases) need the full
 * size.  No reference
 * counterpart: the reference allocates its scratch per call (README.md:105-107
 * describes chunking only for its cuBLAS engine). */
size_t fp64emu_workspace_size_min(int64_t batch, int64_t M, int64_t N, int64_t K,
                                  int nprimes, int use_corr);

/* out[M,N] = A[M,K] @ B[N,K]^T; K up to 128 * 65536, K-segmented past 131071
 * (fp64_emu_cuda/fp64_emu.cu:1479-1579).   fp64_emu_cuda/fp64_emu.cu:1583-1608 */
int fp64emu_mm(double* out, const double* A, const double* B, int64_t M, int64_t N, int64_t K,
               const int32_t* primes /* host */, const int32_t* inv /* host, unused */,
               const int64_t* mu /* host, unused */, int nprimes, int exact, int64_t bits,
               int use_corr, void* workspace, size_t workspace_bytes, fp64emu_stream_t stream);

/* out[M,N] = A[M,K] @ Bt[K,N], Bt consumed in its [K,N] layout (no
 * transpose copy).   fp64_emu_cuda/fp64_emu.cu:1613-1632 */
int fp64emu_mm_nt(double* out, const double* A, const double* Bt, int64_t M, int64_t N, int64_t K,
                  const int32_t* primes, const int32_t* inv, const int64_t* mu, int nprimes,
                  int exact, int64_t bits, int use_corr, void* workspace, size_t workspace_bytes,
                  fp64emu_stream_t stream);

/* out[b,M,N] = A[b,M,K] @ B[b,N,K]^T; K as for fp64emu_mm.
 * fp64_emu_cuda/fp64_emu.cu:1637-1662 */
int fp64emu_bmm(double* out, const double* A, const double* B, int64_t batch, int64_t M, int64_t N,
                int64_t K, const int32_t* primes, const int32_t* inv, const int64_t* mu,
                int nprimes, int exact, int64_t bits, int use_corr, void* workspace,
                size_t workspace_bytes, fp64emu_stream_t stream);

/* out[b,M,N] = A[b,M,K] @ Bt[b,K,N].   fp64_emu_cuda/fp64_emu.cu:1665-1686 */
int fp64emu_bmm_nt(double* out, const double* A, const double* Bt, int64_t batch, int64_t M,
                   int64_t N, int64_t K, const int32_t* primes, const int32_t* inv,
                   const int64_t* mu, int nprimes, int exact, int64_t bits, int use_corr,
                   void* workspace, size_t workspace_bytes, fp64emu_stream_t stream);

/* fp64emu_mm plus phase times in ms, written to the host array
 * times[4] = [sizing+extract, gemms, 0-marker, reconstruct]; synchronizes
 * on the last phase event.   fp64_emu_cuda/fp64_emu.cu:1688-1704 */
int fp64emu_mm_timed(double* out, float* times /* host, 4 floats */, const double* A,
                     const double* B, int64_t M, int64_t N, int64_t K, const int32_t* primes,
                     const int32_t* inv, const int64_t* mu, int nprimes, int exact, int64_t bits,
                     int use_corr, void* workspace, size_t workspace_bytes,
                     fp64emu_stream_t stream);

/* fp64emu_mm_nt that also records five caller-created events on `stream`
 * at the phase boundaries [start, extracted, gemms done, gemms done,
 * reconstructed] (the boundaries of fp64emu_mm_timed) and does not
 * synchronize.  No reference counterpart: it lets a benchmark time each
 * kernel inside its timed loop, on the stream the kernels run on. */
int fp64emu_mm_nt_events(double* out, const double* A, const double* Bt, int64_t M, int64_t N,
                         int64_t K, const int32_t* primes, const int32_t* inv, const int64_t* mu,
                         int nprimes, int exact, int64_t bits, int use_corr, void* workspace,
                         size_t workspace_bytes, fp64emu_stream_t stream,
                         const fp64emu_event_t* events /* host, 5 events */);

/* fp64emu_bmm_nt with the phase events of fp64emu_mm_nt_events (the
 * boundaries of the whole batch's launch chain).  No reference counterpart:
 * the benchmark's per-phase times of batched configs. */
int fp64emu_bmm_nt_events(double* out, const double* A, const double* Bt, int64_t batch, int64_t M,
                          int64_t N, int64_t K, const int32_t* primes, const int32_t* inv,
                          const int64_t* mu, int nprimes, int exact, int64_t bits, int use_corr,
                          void* workspace, size_t workspace_bytes, fp64emu_stream_t stream,
                          const fp64emu_event_t* events /* host, 5 events */);

/* Bytes of the static device scratch of fp64emu_mm_nt_noalloc (64 MiB). */
#define FP64EMU_NOALLOC_SCRATCH_BYTES (64ull << 20)

/* fp64emu_mm_nt without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No reference counterpart.  The
 * first call on a device looks up the scratch's device address
 * (hipGetSymbolAddress); a caller that captures should make one call on
 * that device outside the capture first.  The
 * scratch is a static device array of FP64EMU_NOALLOC_SCRATCH_BYTES that the
 * library holds on every GPU it runs on until the process ends; the call
 * itself allocates nothing.  Products whose full workspace exceeds it run
 * the rows of A in chunks (see fp64emu_workspace_size_min); a product whose
 * smallest workspace exceeds it is rejected with FP64EMU_EWORKSPACE before
 * anything is enqueued.  Every call on one GPU uses that GPU's one array:
 * calls that overlap on one GPU (other streams, other host threads) race
 * and must be serialized by the caller.  The device of `stream` must be the
 * current device.  Results are bit-identical to fp64emu_mm_nt. */
int fp64emu_mm_nt_noalloc(double* out, const double* A, const double* Bt, int64_t M, int64_t N,
                          int64_t K, const int32_t* primes, const int32_t* inv,
                          const int64_t* mu, int nprimes, int exact, int64_t bits,
                          int use_corr, fp64emu_stream_t stream);

/* ---- Workspace map (inspection of intermediates; no reference
 * counterpart: the reference's scratch is private torch tensors).  After a
 * call, the workspace holds that call's sizing outputs, operand planes,
 * residue planes and correction planes at these byte offsets. ---- */
typedef struct {
  int64_t batch, M, N, K;   /* per batch member */
  int nprimes, use_corr;
  int ncorr;                /* int32 correction planes per member: 1 (fused, K <= 65536 and
                               ksplit 1) or 2 */
  int nslab;                /* column-sizing slabs for a [K,N] operand */
  int deep;                 /* K > 131071: the K-segmented form (mm / bmm only) */
  int nseg;                 /* K segments (1 unless deep) */
  int64_t kseg;             /* depth of one segment (K unless deep: 65536) */
  int ksplit;               /* GEMM K-split S: S groups per output tile, each over a K
                               range, with S residue / correction planes summed at
                               reconstruction (1 unless the tiles are few) */
  int nchunk;               /* row chunks of A (1 unless the workspace is smaller than
                               fp64emu_workspace_size; batch 1 only) */
  int64_t chunk_rows;       /* rows of A per chunk (a multiple of 256) */
  int64_t Mp, Np, Kp;       /* padded to the 256-row tile and the 64-deep k tile (of one
                               segment when deep) */
  int64_t planeA_bytes;     /* one residue plane of A for one member: Mp*Kp */
  int64_t planeB_bytes;     /* Np*Kp; the correction plane is twice as deep (2*Kp) */
  int64_t memberA_bytes;    /* all planes of one member: (nprimes + 2*use_corr) * Mp*Kp */
  int64_t memberB_bytes;
  int64_t outplane_bytes;   /* elements of one output plane: Mp*Np.  res8 holds
                               ksplit x batch x P int8 planes, split-major (deep: int32
                               residue sums); corr holds ksplit x batch x ncorr int32
                               planes (deep: one int64 sum plane) */
  size_t off_sftA, off_sftB, off_lgA, off_lgB, off_bits, off_pmax, off_pss;
  size_t off_planesA, off_planesB, off_res8, off_corr, total;
  int gemm_tile_cols;       /* columns of one modular-GEMM output tile: 256, or 128 where
                               128 columns cover N with less padding, for a single
                               modulus in shallow products with many tiles (two work
                               groups per CU), or for shallow products with more moduli
                               and fewer than 256 tiles of 256 x 256 (with more tiles
                               those run slot runs) */
  int gemm_tile_rows;       /* rows of one modular-GEMM output tile: 256, or 128 when
                               128-row tiles cover M with less padding too, or for
                               shallow products of at most 40 tiles of 256 x 256 (not
                               row-chunked) */
  int gemm_run;             /* residue slots one modular-GEMM work group runs back to back
                               for its tile; 1 (one slot per group) except for shallow
                               products (at most 32 k-steps, no K-split) on 256 x 256
                               tiles, of which they have T >= 256 (fewer take 256 x 128
                               or 128 x 128 tiles): one run of all nprimes slots when T
                               is a multiple of 256 (the fused correction slot then
                               leads the run), three runs otherwise (1 when that
                               leaves runs of one) */
  int64_t ext_rowsA;        /* rows of each A plane (per member, per row chunk) that the
                               extraction writes: the operand rows and the zero padding
                               that GEMM tiles read (a multiple of 64, at most the padded
                               row count); rows past it hold unspecified bytes */
  int64_t ext_rowsB;        /* the same for B's plane rows (the columns of B^T) */
  int gemm_split;           /* 1: the modular GEMM runs as split streams (one work group
                               per CU; each XCD's 32 groups walk an equal share of the
                               K-deep (tile, slot) units in blocks of 32, each unit in at
                               most two K ranges, so ksplit is 2) instead of a K-split
                               into rounds of work groups: deep products of 256 x 256
                               tiles for which the planner chose a K-split, with at least
                               eight blocks of units and no last tile column of at most
                               128 columns; 0 otherwise */
} fp64emu_layout_t;

int fp64emu_layout(int64_t batch, int64_t M, int64_t N, int64_t K, int nprimes, int use_corr,
                   fp64emu_layout_t* out /* host */);

/* ---- Measurement helper (not on the product path): double-double GEMM
 * C = A @ B^T (A [M,K], B [N,K], row-major), hi/lo outputs [M,N].  The GPU
 * form of the reference's correct-bits oracle bench/accuracy.py:21-50
 * (dd_matmul_nt), accumulating each dot product in ~106-bit arithmetic. */
int fp64emu_ddgemm_nt(double* hi, double* lo, const double* A, const double* B, int64_t M,
                      int64_t N, int64_t K, fp64emu_stream_t stream);

/* ---- Ceiling probes (measurement helpers, not on the product path; no
 * reference counterpart).  They measure the rates this part attains, which
 * the benchmark reports beside the datasheet peaks. ---- */

/* The modular GEMM's inner loop, on `groups` work groups of 4 waves (one
 * group per CU), `steps` steps of 64 v_mfma_i32_16x16x64_i8 per wave in the
 * GEMM's order, over two 32 KiB stages of int8 fragments at `src` (64 KiB,
 * A tile then B tile per stage, in the planes' fragment order).
 *   mode 0: fragments held in registers (no memory traffic);
 *   mode 1: the next step's fragments read from the GEMM's 4-stage LDS ring,
 *           with its per-step wait and barrier;
 *   mode 2: mode 1 plus the GEMM's global->LDS copies (from `src`, which the
 *           L2 caches hold).
 * acc_out (256 KiB) receives group 0's accumulators: the sum over the steps
 * of each step's stage products, as [wave][x][y] blocks of 256 int32 (lane
 * l's value v of the 16 x 16 block at 4 l + v: row 4 (l / 16) + v, column
 * l % 16).  clocks[4 * g .. 4 * g + 3] receive group g's shader-clock counter
 * (s_memtime) and 100 MHz real-time counter (s_memrealtime) at the start and
 * the end of its loop: [clk0, clk1, rt0, rt1]. */
int fp64emu_probe_mfma(int32_t* acc_out, unsigned long long* clocks, const int8_t* src,
                       int64_t groups, int64_t steps, int mode, fp64emu_stream_t stream);

/* HBM streaming over n doubles (n even, >= 2048; 16-byte aligned buffers):
 * mode 0 reads src (the per-group sums go to dst[0 .. min(n / 2048, 4096))),
 * mode 1 writes dst = 1.0 (src unused), mode 2 writes dst = -src. */
int fp64emu_probe_stream(double* dst, const double* src, int64_t n, int mode,
                         fp64emu_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FP64EMU_H */
