// internal.h -- shared declarations between the KMeans kernels and the
// host runtime of libskmetal_hip.so (gfx950 / MI355X).
//
// Device data layout for one Lloyd problem (n rows, d features, k clusters):
//   X       fp32 [n x ld]   column-centred rows, ld = round_up(d, 4), pad = 0
//   C[2]    fp32 [k x ld]   centres (double-buffered: old -> new each step)
//   cnorm   fp32 [k]        ||c_j||^2 of the current centres
//   labels  int32 [n]
// Everything stays resident in HBM for the whole fit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace skm {

// Per-fit loop state, resident in device memory.  Every kernel of the
// Lloyd loop reads `done` first and returns at once when it is non-zero,
// so a whole batch of iterations can be enqueued without host round trips.
struct LoopState {
    int done;          // 0 run, 1 strict label convergence, 2 shift <= tol,
                       // 3 empty cluster: host relocation needed at `halt_iter`
    int n_iter;        // sklearn's n_iter_ (iterations completed)
    int chg[2];        // labels changed by the E-step of iteration i: chg[i & 1]
    int last_changed;  // changes of the last decided iteration
    int halt_iter;     // iteration index at which `done` was set
    int n_empty;       // empty clusters found by the last finalise
    unsigned reloc_ctr;  // k_reloc: blocks done with their rows (the last resets it)
    int reloc_iter;      // iteration whose empty clusters k_reloc relocated (-1: none)
    int empty_cnt[2];    // clusters k_finalize_cols of iteration i found empty: empty_cnt[i & 1]
    double shift_tot;  // sum_j ||c_j_new - c_j_old||^2 of the last step
    double inertia;    // result of the last row-distance reduction
    // fused steps (k <= 64): bit j set when a block of iteration i's fused
    // kernel labelled a row j: present[i & 1]
    unsigned long long present[2];
};

enum StepFlags : int {
    kStopStrict = 1,   // stop when an E-step changes no label (sklearn rule)
    // the shift rule is sqrtf(max_j ||c_j_new - c_j_old||^2) < tol (skmetal's
    // KMeansBridge.swift:306-310) instead of sum_j ||..||^2 <= tol (sklearn's)
    kStopMaxShift = 2,
};

// The loop's shift rule: sum of squared shifts <= tol (sklearn), or, with
// kStopMaxShift, the largest shift's fp32 root < tol (skmetal's reference
// loop).  tol < 0: no shift rule (fixed iterations).
__host__ __device__ inline bool shift_rule_stops(int flags, double tol, double sum_sq, float max_sq)
{
    if (tol < 0.0) return false;
    if (flags & kStopMaxShift) return sqrtf(max_sq) < (float)tol;
    return sum_sq <= tol;
}

// ---- kernel launchers (kmeans_kernels.hip) -------------------------------
// All return hipSuccess or the launch error; all enqueue on `s`.

struct AssignArgs {
    const float* X; long n; int ld;
    const float* C; const float* cnorm; int k;
    int* labels;
    LoopState* state;      // nullable: no early exit
    int* changed;          // nullable: compare with previous labels, add the changes here
    char* img;             // k_assign3 only: [assign3_image_bytes(k, ld)] the centres' staged image
    // k_assign3 only, nullable: the inertia of the new labels, fp64 block
    // totals ([num_cu] at most; their number to *inert_blocks) of the rows'
    // squared distances to their centres (direct form, as k_rowdist); d is
    // the row length these use
    double* inert = nullptr;
    int* inert_blocks = nullptr;
    int d = 0;
    // k_assign3 only, nullable: each row's minimum ||c||^2 - 2 x.c (as
    // FusedArgs::emin), for the relocation's candidate search
    float* emin = nullptr;
};
hipError_t launch_assign(const AssignArgs& a, int num_cu, hipStream_t s);
// The same E-step on bf16 MFMAs over the exact three-part bf16 split of x
// and c (k_assign3); assign3_ready(d, k) = 1 when it applies to the shape
// (sets its LDS attributes).  The data must be in the split's range
// (split_range_ok).
int assign3_ready(int d, int k);
// Bytes of k_assign3's centre image (written by launch_assign3 before the E-step).
size_t assign3_image_bytes(int k, int ld);
hipError_t launch_assign3(const AssignArgs& a, int num_cu, hipStream_t s);
// The three-part bf16 split is exact for finite values of magnitude >= 2^-103,
// and the E-step's smallest kept part products stay normal fp32 numbers when
// the data's largest magnitude is 0 or at least 2^-50.
inline bool split_range_ok(float absmax) { return absmax == 0.f || (absmax >= 0x1p-50f && absmax <= 0x1p+60f); }

// Fused E-step + per-cluster sums (k <= 64, d <= 100).
struct FusedArgs {
    const float* X; long n; int ld;
    const float* C; const float* cnorm; int k;
    int* labels;
    float* psum;           // [blocks x k x ld]
    int* pcnt;             // [blocks x k]
    LoopState* state;      // required: early exit
    int blocks;
    int* changed;          // this E-step's changed labels (added)
    // decide = 1: every block first evaluates the stopping rules of the
    // previous step (iteration iter - 1) from the finalize's chunk partials,
    // as k_finalize_loop does, and block 0 records the decision; the step's
    // ||c||^2 then come from those partials instead of `cnorm`
    int decide; int iter; double tol; int flags;
    const double* part; int nch; const int* counts; const int* prev_changed;
    float* cnorm_out; float* shift_sq;
    // split = 1: k_fused3 (E-step and sums on bf16 MFMAs over the exact
    // three-part split); see fused3_ready
    int split = 0;
    // k_fused3, nullable: each row's minimum ||c||^2 - 2 x.c (the distance to
    // its new centre less ||x||^2), for the relocation's candidate search
    float* emin = nullptr;
};
// Row stride (floats) X must have for the fused kernel, or 0 when (d, k) does
// not qualify; the pad columns are zero.
int fused_ld(int d, int k);
// Number of blocks (= partials) of the fused kernel for n rows of stride ld.
int fused_blocks(long n, int ld, int k, int num_cu);
// 1 when the split fused kernel exists for (k, ld) and fits in LDS (sets its
// LDS attribute); the data must still be in the split's range.
int fused3_ready(int k, int ld);
hipError_t launch_fused3(const FusedArgs& a, hipStream_t s);
hipError_t launch_fused(const FusedArgs& a, hipStream_t s);

struct UpdateArgs {
    const float* X; long n; int ld; int d;
    const int* labels; int k;
    float* psum;           // [R x k x ld]
    int* pcnt;             // [R x k]
    LoopState* state;
};
struct UpdateGeom { int R; int G; int Z; int cg; int nslots; int ncp; int W; long rows_per_range; int threads; size_t lds; };
UpdateGeom update_geometry(long n, int d, int k, int num_cu);
hipError_t launch_update(const UpdateArgs& a, const UpdateGeom& g, hipStream_t s);

// Sorted update for the generic path: rows are ordered by label with a
// counting sort (per-range histograms, scan, scatter), then chunks of the
// sorted order are summed segment by segment; cluster j's partial sums are
// the records rec_off[j] .. rec_off[j] + rec_cnt[j] - 1 (chunk order).
struct SortGeom {
    bool on = false;
    int wr = 0;            // rows per range (one wave each)
    int nw = 0;            // ranges
    int nseg = 0;          // scan segments of kSortSeg ranges
    int B = 0;             // sorted rows per chunk
    long nchunks = 0;
    int G = 0;             // threads per chunk group (covers the row's columns)
    long max_records = 0;  // k + nchunks
};
constexpr int kSortSeg = 32;
SortGeom sort_geometry(long n, int d, int ld, int k);
struct SortArgs {
    const float* X; long n; int ld; int d;
    const int* labels; int k;
    int* hist;             // [nw x k]: range histograms, then range offsets
    int* segsum;           // [nseg x k]
    int* counts;           // [k]  rows per cluster
    int* start;            // [k]  first sorted position of cluster j
    int* rec_off;          // [k]  first record of cluster j
    int* rec_cnt;          // [k]  records of cluster j
    int* perm;             // [n]  row ids in sorted order
    int* slab;             // [n]  labels in sorted order
    float* rec;            // [max_records x ld]
    LoopState* state;
};
hipError_t launch_sorted_update(const SortArgs& a, const SortGeom& g, hipStream_t s);

struct FinalizeArgs {
    const float* psum; const int* pcnt; int R; int k; int d; int ld;
    // record mode (sorted update): cluster j's partials are the records
    // rec_off[j] .. + rec_cnt[j] of psum and its count is cnt_in[j]; null
    // otherwise (partials r*k + j for r < R, counts summed from pcnt)
    const int* rec_off; const int* rec_cnt; const int* cnt_in;
    const float* C_old; float* C_new; float* cnorm;
    double* sums;          // [k x ld] fp64 totals (kept for the relocation path)
    int* counts;           // [k]
    double* part;          // [k x nch x 2]
    float* shift_sq;       // [k]
    LoopState* state;
    int iter; double tol; int flags;
    int cw;                // columns per finalize block: finalize_cols(R)
    const int* chg_cur;    // changes of this step's E-step
    int* chg_next;         // cleared for the next step's E-step
    int after_reloc = 0;   // loop decision right after a relocation: empty
                           // clusters do not stop the loop, every ||c||^2 is set
};
// Per-(cluster, column chunk) totals, then (with_loop) the loop decision.
hipError_t launch_finalize(const FinalizeArgs& a, hipStream_t s, bool with_loop);
// The loop decision alone (after a fused step whose successor is not enqueued).
// nch: the chunk count the partials were written with (0: that of a.R).
hipError_t launch_finalize_loop(const FinalizeArgs& a, hipStream_t s, int nch = 0);
// A finalize block is 256 threads = 8 float4 columns (32 columns) x 32
// partial-sum lanes.
inline int finalize_cols(int R)
{
    (void)R;
    return 32;
}
inline int finalize_col_chunks(int d, int R) { const int cw = finalize_cols(R); return (d + cw - 1) / cw; }

struct RowDistArgs {
    const float* X; long n; int ld; int d;
    const float* C; int k; const int* labels;  // rows with a label outside [0, k) count 0
    float* out_rows;       // nullable: per-row squared distance
    double* block_part;    // [rowdist_grid(n)]: the blocks' totals
    LoopState* state;      // receives `inertia`
};
constexpr int kRowDistBlocks = 512;  // largest row-distance grid
int rowdist_grid(long n);            // block totals to allocate for n rows
// Row distances and their fixed-order total (k_rowdist or k_rowdist_slab,
// then k_rowdist_total adds the block totals in block order).
hipError_t launch_rowdist(const RowDistArgs& a, hipStream_t s);
// The fixed-order total of nb fp64 block totals into state->inertia
// (k_rowdist_total).
hipError_t launch_inertia_total(const double* parts, int nb, LoopState* state, hipStream_t s);

// Device relocation of up to kMaxReloc empty clusters at once (see
// kmeans_kernels.hip); more go through the host.
constexpr int kMaxReloc = 64;
constexpr int kRelocBlocks = 256;   // candidate blocks
constexpr int kRelocCW = 64;        // columns per k_finalize_sums block
struct RelocArgs {
    const float* X; long n; int ld; int d; int k;
    const int* labels;
    const float* dist;     // [n] k_rowdist's per-row distances to the old centres
    float* cand_d;         // [kRelocBlocks x E]
    long* cand_i;          // [kRelocBlocks x E]
    double* sums;          // [k x ld] fp64 totals, updated in place
    int* counts;           // [k], updated in place
    int* amax;             // [1] heaviest cluster after the moves
    const float* C_old; float* C_new;
    double* part;          // [k x nch x 2], nch = ceil(d / kRelocCW)
};
// E = number of empty clusters (1 <= E <= kMaxReloc).
hipError_t launch_relocate(const RelocArgs& a, int E, hipStream_t s);

// In-stream relocation (k_reloc, launched after every step's
// k_finalize_cols): when step `iter` left 1..kMaxReloc clusters empty, the
// rows farthest from their centres move to them and the centres and chunk
// partials of the clusters involved are redone, before the step's loop
// decision; with no empty cluster the kernel returns at once.
struct InRelocArgs {
    const float* X; long n; int ld; int d; int k;
    const int* labels;     // step iter's labels
    const float* C_old;    // the centres those labels were taken against
    float* C_new;          // the step's new centres (k_finalize_cols's, rewritten)
    double* sums;          // [k x ld] the step's fp64 sums (updated in place)
    int* counts;           // [k] (updated in place)
    double* part;          // [k x nch x 2] the finalize's chunk partials (rewritten)
    int nch;               // chunks of finalize_cols(.) columns
    float* dist;           // [n] scratch: row distances
    float* cand_d;         // [kRelocInlineBlocks x kMaxReloc]
    long* cand_i;          // [kRelocInlineBlocks x kMaxReloc]
    int* amax;             // [1]
    LoopState* state; int iter;
    // nullable (both or neither): ||x||^2 per row and the E-step's row
    // minima (FusedArgs::emin, AssignArgs::emin) of these labels; with them
    // the blocks compute direct-form distances only for rows whose
    // approximate distance xnorm + emin lies near the top (rows of at most
    // 128 floats)
    const float* xnorm = nullptr;
    const float* emin = nullptr;
};
constexpr int kRelocInlineBlocks = 256;  // grid of k_reloc / k_finalize_reloc (one block per CU: their LDS)
constexpr int kRelocLdsRows = 4096;      // a block's row distances kept in LDS (more rows: InRelocArgs::dist)
constexpr int kRelocCandBlocks = kRelocInlineBlocks > kRelocBlocks ? kRelocInlineBlocks : kRelocBlocks;  // candidate list rows
hipError_t launch_reloc_inline(const InRelocArgs& a, hipStream_t s);
// The fused step's k_finalize_cols and k_reloc in one launch (k <= 64, at
// most kRelocInlineBlocks finalize chunks, no update records): the empty
// clusters come from the fused kernel's presence bits.
hipError_t launch_finalize_reloc(const FinalizeArgs& f, const InRelocArgs& a, hipStream_t s);
// Writes v to *st (a one-thread kernel: no host synchronisation).
hipError_t launch_state_reset(LoopState* st, const LoopState& v, hipStream_t s);

// Greedy k-means++ seeding (plusplus_kernels.hip): sklearn's _kmeans_plusplus
// with unit weights and the random draws made by the caller.
constexpr int kPPRows = 256;        // rows per k_pp_dist block (one per thread)
constexpr int kPPMaxTrials = 64;    // largest n_local_trials
struct PPArgs {
    const float* X; long n; int ld;
    int k;
    int T;                 // n_local_trials (candidates per centre after the first)
    int nb;                // k_pp_dist blocks = ceil(n / kPPRows)
    float* D[2];           // [T x n] min(closest, distance to candidate t), by centre parity
    double* P[2];          // [T x nb] per-block fp64 sums of D[.][t]
    double* pfx;           // [nb] inclusive prefix of the chosen candidate's block sums
    long* cand;            // [T] candidate rows of the centre being drawn (cand[0] = first row at start)
    long* idx;             // [k] chosen rows
    int* best;             // [k] chosen candidate of each centre
    double* pot;           // [k] potential after each centre (fp64 total)
    const double* U;       // [(k - 1) x T] uniforms in [0, 1), in sklearn's draw order
    float* centers;        // [k x ld] the chosen rows of X
    float* mind;           // [n] k-means||: running minimum distance over the candidates so far
    int mind_reset;        // k-means||: 1 = start the minimum from +inf
    int cus;               // compute units of the device (the distance kernel's grid)
    double* ctab;          // [ld / 4][T][4] the drawn candidates' values as fp64 (pp_rows_path only; else null)
    double* xxn;           // [n] ||x||^2 in fp64, written by the first centre's distances (with ctab; else null)
    double* ccn;           // k-means||: [m] the candidates' ||c||^2 (with ctab, [ld / 4][m][4]; else null)
};
// Whether k_pp_dist's rows path (and so a.ctab) serves T candidates of rows of ld floats.
inline bool pp_rows_path(int T, int ld) { return T <= 8 && ld <= 128; }
// Whether the k-means|| rounds' rows path (a.ctab, a.ccn) serves rows of ld floats.
inline bool pp_rows_min_path(int ld) { return ld <= 128; }
// Candidate distances of centre c (c = 0: the first row alone).
hipError_t launch_pp_dist(const PPArgs& a, int c, hipStream_t s);
// k-means||: mind[row] = min(mind[row] (or +inf with mind_reset), distance to
// each of the m candidate rows cand[0 .. m-1]), distances in the same form.
hipError_t launch_pp_mindist(const PPArgs& a, int m, hipStream_t s);
// Pick centre c - 1 among its candidates; for c < k draw centre c's candidates.
hipError_t launch_pp_select(const PPArgs& a, int c, hipStream_t s);

// Weighted draws without replacement in numpy's RandomState.choice form
// (sample_kernels.hip): probabilities p = fp32(w / sum(w)) as fp64, then per
// pass of uniforms the rows searchsorted(cumsum(p) / cumsum(p)[-1], u, "right").
constexpr int kWSBlock = 8192;  // numpy reduces a contiguous fp32 array one 8192-element buffer at a time
constexpr int kWSChunk = 2048;  // rows per search chunk
struct WSArgs {
    const float* w; long n;     // weights (nullptr: unit weights)
    float floor;                // numpy maximum(w, floor), NaN kept
    float* bsum;                // [ws_blocks(n)] fp32 pairwise sum of each 8192-weight block
    float* total;               // [1] fp32 sum of the weights, numpy's order
    double* p;                  // [n] probabilities (fp64 of the fp32 quotient)
    double* ctot;               // [ws_chunks(n)] fp64 sum of each chunk of p
    int* cnz;                   // [ws_chunks(n)] rows with p > 0 per chunk
    double* pfx;                // [ws_chunks(n) + 1] chunk sums' running total, pfx[0] = 0
    long long* nnz;             // [1] rows with p > 0
    double* cst;                // [ws_chunks(n) + 1] numpy's cumsum before each chunk, then the total (exact search)
    int* cseq;                  // [ws_chunks(n)] 1: the chunk's sums come from a walk in row order
    const double* u; int m;     // this pass's uniforms
    double dmin;                // the certified search's least margin (0; larger sends more draws to the exact search)
    const long* zero; int nz;   // rows whose p is zeroed before the pass
    long* out;                  // [m] picked rows
    int* unsure;                // [m] 1: the certified search left the draw to the exact search
};
int ws_blocks(long n);
int ws_chunks(long n);
// p, chunk sums, prefix and the non-zero count from the weights.
hipError_t launch_ws_prepare(const WSArgs& a, hipStream_t s);
// p[zero[0 .. nz-1]] = 0, then chunk sums and prefix again.
hipError_t launch_ws_zero(const WSArgs& a, hipStream_t s);
// Certified search of the m uniforms: out, unsure.
hipError_t launch_ws_search(const WSArgs& a, hipStream_t s);
// numpy's sequential cumsum (exactly, per chunk), then the search of the
// unsure draws (all != 0: every draw).
hipError_t launch_ws_exact(const WSArgs& a, int all, hipStream_t s);

// KMeans.transform (transform_kernels.hip): out[i, j] = ||x_i - c_j|| in
// scikit-learn's fp32 form (fp64 expanded distance, fp32 cast, clamp, sqrt).
struct TransformArgs {
    const float* X; long n; int ld;    // rows, stride ld (pad columns 0)
    const float* C; int k;             // centres [k x ld]
    double* cc;                        // [k] fp64 ||c||^2 (written first)
    float* out;                        // [n x k]
    double* cfrag = nullptr;           // transform_mm_path: [ceil(k / 16) 16 ld] the centres as fp64 MFMA fragments
    int cus = 0;                       // compute units of the device
};
// Whether KMeans.transform takes the fp64 matrix-core kernel (rows of <= 128 floats).
inline bool transform_mm_path(int ld) { return ld <= 128; }
hipError_t launch_transform(const TransformArgs& a, hipStream_t s);

hipError_t launch_colsum(const float* X, long n, int ld, int d, double* part, int nblk, hipStream_t s);
int colsum_grid(long n);
hipError_t launch_colmean(const double* part, int nblk, long n, int d, float* mean, hipStream_t s);
hipError_t launch_center(float* X, long n, int ld, int d, const float* mean, hipStream_t s);
// max |x| over count floats (NaN as +inf) into *out as float bits
hipError_t launch_absmax(const float* X, long count, unsigned* out, hipStream_t s);
// out[r] = ||x_r||^2 (fp32) of the n rows of stride ld (d features)
hipError_t launch_rownorm(const float* X, long n, int ld, int d, float* out, hipStream_t s);
hipError_t launch_cnorm(const float* C, int k, int ld, float* cnorm, hipStream_t s);

}  // namespace skm
