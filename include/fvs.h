/*
 * fvs.h - C ABI of libfvs.so, the MI355X (gfx950) kernels of the FanarVSE batched search path
 * (route -> int8 cell-residual stage 1 with threshold-and-emit -> LUT stage 2 with error bars
 * -> exact fp16 refinement of the ambiguous candidates).
 *
 * Conventions shared by every entry point
 *   - Pointers are device pointers unless a comment says otherwise (the refine entry point also
 *     accepts a pinned, device-mapped host pointer for the fp16 rows).
 *   - Sizes are plain integers; `stream` is a hipStream_t passed as void* (torch's
 *     torch.cuda.current_stream().cuda_stream), the way the reference hands torch's stream to
 *     its CUDA twin (throughput/civf8.py:89-91).
 *   - Every call returns 0 on success, a positive hipError_t if a launch failed, or a negative
 *     FVS_E_* code when an argument is out of range (nothing is launched then).
 *   - The library never allocates, frees or synchronises: every buffer, scratch included, is
 *     owned by the caller, so a whole search can be captured in one hipGraph. Calls are reentrant
 *     (no mutable global state); calls that share an output buffer must be ordered by the caller.
 *   - fp16 data is passed as uint16_t (IEEE binary16 bit patterns).
 *
 * Determinism: every floating-point result has one canonical operation order, written next to
 * each entry point; the CPU checker under oracle/ follows the same order, so results are
 * bit-identical for identical inputs. The order in which the emit pass appends candidates is
 * not deterministic (atomics), as in the reference; everything read back from the buffer is.
 */
#ifndef FVS_H
#define FVS_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FVS_ABI_VERSION 2

#define FVS_OK 0
#define FVS_E_ARG (-1)      /* an argument is out of its documented range            */
#define FVS_E_SHAPE (-2)    /* a shape the kernels do not support (R, d, tiers, ...) */
#define FVS_E_CAPACITY (-3) /* a per-workgroup capacity is exceeded (K, n_p, cell)   */

/* Maximum tiers of the refinement code (the reference asserts <= 6: src/tiered_fused.py:55). */
#define FVS_MAX_TIERS 8

/* ABI version (FVS_ABI_VERSION) and a static description of an error code. */
int fvs_abi_version(void);
const char *fvs_error_string(int code);

/* Fill n 32-bit words with `value` (graph-capturable replacement for hipMemsetAsync). */
int fvs_fill_u32(void *dst, int64_t n, uint32_t value, void *stream);

/* Matrix-core calibration (no reference counterpart: the achievable-peak measurement that bench.py reports
 * beside the published one). `blocks` workgroups of 256 threads; every wave runs `iters` rounds of four
 * independent 4-step v_mfma_i32_16x16x64_i8 chains on register operands (2 * 16 * 16 * 16 * 64 int8 ops per
 * round) and writes one checksum to out[wave] (out holds blocks * 4 int32). */
int fvs_calib_mfma(int32_t blocks, int32_t iters, int32_t *out, void *stream);

/*
 * The latency path's host result in one launch: out i64 [B, k+1] = [ok[q] | I[q][0..k)] (ok u8 [B],
 * I i32 [B, k]). out may be pinned host memory: the launch writes it directly, and the values are
 * visible to the host once the stream has been synchronised. Replaces the int64 casts, the
 * concatenation and the device-to-host copy of the flags and ids that src/engine_cell.py:152-165
 * performs after its graph (ok.cpu(), I.cpu()).
 */
int fvs_pack_ids(const uint8_t *ok, const int32_t *I, int64_t B, int32_t k, int64_t *out, void *stream);

/*
 * The default engine's three dense products for a batch of at most 8 queries, in one launch. Replaces the
 * library products Qb @ s1["W1"] and Qb.half() @ s1["means16"].T of src/engine_cell.py:76,79 and the
 * stage-2 query rotation Qb @ VP of src/tiered_fused.py:57 at small batch: Qr f32 [B, R] = Q @ W1T^T, QM fp16 [B, NC] = fp16(fp16(Q) @ M16^T) (f32
 * sums), Zq f32 [B, D] = Q @ VPT^T, and qc f32 [B] = <Q, c> exactly as fvs_query_prep computes it (the
 * reference's QC = Qb @ s1["c"], src/engine_cell.py:76). W1T f32 [R, d], M16 fp16 [NC, d] and VPT f32 [D, d]
 * are row-major (the transposes of W1 and VP, made once). Each product output is one wave's dot: per
 * lane, 4-element slices in k order, then the xor butterfly 32..1. d must be a multiple of 4.
 */
int fvs_dense_small(const float *Q, int64_t B, int32_t d, const float *W1T, int32_t R, float *Qr, const uint16_t *M16,
                    int32_t NC, uint16_t *QM, const float *VPT, int32_t D, float *Zq, const float *c, float *qc,
                    void *stream);

/*
 * Query code (a6) plus the global-centre term and the fp16 copy of the queries.
 * Replaces throughput/enginei8.py:38 (qs = max|z|/127; q8 = round(z/qs), with z = Qb @ Vr computed by
 * the caller's fp32 BLAS as in the reference), throughput/enginei8.py:62 (QC = Qb @ c) and the
 * Qb.half() casts at :67 and s2lut.py:122.
 *   Q  f32 [B, d] row-major; z f32 [B, R] = Q @ Vr; c f32 [d]
 *   q8 i8 [B, R]; qs f32 [B]; qc f32 [B]; qh fp16 [B, d]
 * Canonical order: qs = max(max_j |z[j]|, 1e-12f) / 127.0f; q8[j] = clamp(rintf(z[j] / qs), -127, 127);
 *   qc = (float) of the double sum of the (exact) products (double)Q[k]*(double)c[k]: lane l = k % 64
 *   accumulates its products in k order, then lane[l] += lane[l ^ o] for o = 32, 16, 8, 4, 2, 1.
 * R must be 256; d must be a multiple of 8.
 */
int fvs_query_prep(const float *Q, int64_t B, int32_t d, const float *z, int32_t R, const float *c,
                   int8_t *q8, float *qs, float *qc, uint16_t *qh, void *stream);

/*
 * fvs_query_prep with the projection computed by the library: z f32 [B, R] = Q @ Vr (Vr f32 [d, R],
 * row-major), each output a sequential fmaf chain over k = 0 .. d - 1 from +0 (the order of fvs_build_codes'
 * projection, so the oracle reproduces z bit for bit), written to z; then q8, qs, qc and qh exactly as
 * fvs_query_prep computes them from that z. Replaces the fp32 BLAS product Qb @ Vr of
 * throughput/enginei8.py:38 together with the code, the centre term (:62) and the casts (:67).
 * R must be 256; d must be a multiple of 8.
 */
int fvs_query_code(const float *Q, int64_t B, int32_t d, const float *Vr, int32_t R, const float *c, float *z,
                   int8_t *q8, float *qs, float *qc, uint16_t *qh, void *stream);

/*
 * int8 cell-residual codes of the base set (a3). Replaces build_codes, throughput/enginei8.py:19-27.
 *   X16 fp16 [n_ids, d] in id order; order i32 [N] (sorted position -> id);
 *   cell i32 [N] (cell of each sorted position); means16 fp16 [NC, d]; Vr f32 [d, R]
 *   Z i8 [N, R] in sorted order; zs f32 [N]
 * Canonical order: x[k] = (float)X16[order[n]][k] - (float)means16[cell[n]][k] (one f32 subtraction);
 *   z[j] = fmaf(x[k], Vr[k][j], z[j]) for k = 0..d-1 from +0 (a build-time kernel, so every output is
 *   one sequential chain); then the quantisation of fvs_query_prep.
 */
int fvs_build_codes(const uint16_t *X16, const int32_t *order, const int32_t *cell, int64_t N, int32_t d,
                    const uint16_t *means16, const float *Vr, int32_t R, int8_t *Z, float *zs, void *stream);

/*
 * Routing top-n_p (a7). Replaces `probe = QM.topk(nprobe, 1).indices` (throughput/enginei8.py:68).
 *   QM fp16 [B, NC]; probe i32 [B, nprobe], each row sorted by (QM value descending, cell ascending);
 *   -0 and +0 compare equal. nprobe <= min(NC, 4096), NC <= 16384.
 */
int fvs_route_topk(const uint16_t *QM, int64_t B, int32_t NC, int32_t nprobe, int32_t *probe, void *stream);

/*
 * (query, cell) pairs grouped by cell (a8). Replaces pairs_fast (throughput/enginei8.py:11-16) with
 * scale = |m_c| (the NROUTE branch, :47).
 *   probe i32 [B, npr] (only the first n columns are used; a row holds distinct cells);
 *   QM fp16 [B, NC]; mnorm f32 [NC] or NULL (scale 1)
 *   ccnt i32 [NC]  number of pairs of each cell      coff i32 [NC]  exclusive prefix of ccnt
 *   scratch        at least fvs_pairs_scratch_bytes(B, NC) bytes, 16-byte aligned (cell-major probe-rank and score matrices)
 *   qid i32 [B*n]  query of each pair, cell-major, queries ascending inside a cell (the stable-sort order)
 *   qrank i32 [B*n] rank of the cell in the query's probe row     qcp f32 [B*n] = (float)QM[q][c] * mnorm[c]
 *   qadd f32 [B] or NULL: when given, qcp += qadd[q] (the projected-means variant of the host-resident engine,
 *   host_resident/space_x.py:33-36, where QM holds q.(m_c - c) in the stage-1 subspace and qadd = <q, c>)
 */
int64_t fvs_pairs_scratch_bytes(int64_t B, int32_t NC);
int fvs_pairs(const int32_t *probe, int64_t B, int32_t npr, int32_t n, int32_t NC, const uint16_t *QM,
              const float *mnorm, const float *qadd, int32_t *ccnt, int32_t *coff, void *scratch, int64_t scratch_bytes,
              int32_t *qid, int32_t *qrank, float *qcp, void *stream);

/*
 * fvs_pairs without a scratch argument, for callers that cannot allocate device memory (code under graph
 * capture, serving loops, harnesses that forbid hipMalloc). No counterpart in the reference: its pair
 * lists come from torch ops. Same inputs, outputs and results as fvs_pairs; the rank and score matrices
 * live in a static device array of FVS_PAIRS_NOALLOC_SCRATCH bytes that the library holds on each device
 * it runs on until the process ends, so fvs_pairs_scratch_bytes(B, NC) must not exceed it (FVS_E_CAPACITY
 * otherwise: 32 MiB covers B <= 2048 at NC = 4096). The call allocates and frees nothing. Every call on a
 * device shares that device's array and overwrites what it reads (nothing needs clearing between calls):
 * calls that overlap on one device race, so callers serialise them (one stream, or events).
 */
#define FVS_PAIRS_NOALLOC_SCRATCH (32 << 20)
int fvs_pairs_noalloc(const int32_t *probe, int64_t B, int32_t npr, int32_t n, int32_t NC, const uint16_t *QM,
                      const float *mnorm, const float *qadd, int32_t *ccnt, int32_t *coff, int32_t *qid,
                      int32_t *qrank, float *qcp, void *stream);

/*
 * Both pair lists of one search batch from one pass: the first-pass list of the first n1 probe columns
 * (ccnt1, coff1, qid1, qrank1, qcp1 over B*n1 pairs) and the emit list of all npr columns (ccnt, coff,
 * qid, qrank, qcp over B*npr pairs), each exactly as fvs_pairs gives it. Replaces the two pairs_fast
 * calls of stage1_i8 (throughput/enginei8.py:48,55); scratch as for fvs_pairs. npr <= 65535.
 */
int fvs_pairs2(const int32_t *probe, int64_t B, int32_t npr, int32_t n1, int32_t NC, const uint16_t *QM,
               const float *mnorm, const float *qadd, void *scratch, int64_t scratch_bytes, int32_t *ccnt1,
               int32_t *coff1, int32_t *qid1, int32_t *qrank1, float *qcp1, int32_t *ccnt, int32_t *coff,
               int32_t *qid, int32_t *qrank, float *qcp, void *stream);

/*
 * The reference's operator seam for the int8 stage-1 scan (a9, a11), argument for argument:
 * civf8.launch(mode, P, q8, qs, qid, coff, ccnt, pcell, pblk, ps, pe, Z, zs, qcp, t0, cnt, bval, bpos, bmc,
 * CAP, MB) (throughput/civf8.py:89-91, called by EngineI8.stage1_i8 at throughput/enginei8.py:49-52,58),
 * which the Triton pair _first8c/_emit8c (throughput/ivf8c_kern.py:2-36) also implements.
 *   P work items (pcell, pblk, ps, pe) = _static_blocks (src/s1cell.py:161-168): item p covers the rows
 *   [32 pblk, 32 pblk + 32) of [ps, pe), the rows of cell pcell; Z i8 [N, 256], zs f32 [N] in the same row
 *   order; (qid, coff, ccnt, qcp) = pairs_fast's lists (throughput/enginei8.py:11-16): the pairs of cell c
 *   are qoff = coff[c] .. qoff + ccnt[c] - 1 with query qid[pair] and centre term qcp[pair].
 *   For every pair of the item's cell: acc = sum_j q8[q][j] * Z[n][j] (int32), est = fmaf((float)acc * qs[q],
 *   zs[n], qcp[pair]) for the rows n of the item.
 *   mode 0: bmc[pair * MB + pblk - ps / 32] = max over the item's rows (fmaxf from -1e30); other entries are
 *     left as they are (the caller pre-fills -1e30, as the reference does). t0, cnt, bval, bpos unused.
 *   mode 1: every (q, n) with est >= t0[q] increments cnt[q]; the first CAP of a query are stored at
 *     bval[q*CAP + idx], bpos[q*CAP + idx] = n (any order). cnt zeroed by the caller. bmc unused.
 * R is 256, as the reference's kernel fixes it. One wave per item: a compatibility entry; the engine's own
 * path (fvs_i8_scan below) groups a cell's blocks into items of eight, which the one-block list cannot
 * express, and writes block maxima by query instead of by pair.
 */
int fvs_i8_scan_civf8(int32_t mode, int32_t P, const int8_t *q8, const float *qs, const int32_t *qid,
                      const int32_t *coff, const int32_t *ccnt, const int32_t *pcell, const int32_t *pblk,
                      const int32_t *ps, const int32_t *pe, const int8_t *Z, const float *zs, const float *qcp,
                      const float *t0, int32_t *cnt, float *bval, int32_t *bpos, float *bmc, int32_t CAP, int32_t MB,
                      void *stream);

/*
 * int8 stage-1 scan on MFMA (a9, a11), the engine's grouped form of fvs_i8_scan_civf8 (same estimates and
 * emitted sets; throughput/civf8.py:89-91, throughput/ivf8c_kern.py:2-36), plus qrank/n1 so that the first
 * pass writes each query's block maxima straight into its own row.
 *   Work item p < P: a cell and consecutive rows of it (pcell, prow, ps, pe: the cell, the item's first
 *   row, and the cell's first and end row). Mode 0: the item covers rows [max(prow, ps), min(prow + 128,
 *   pe)) as four 32-row blocks starting at prow; prow is a multiple of 32 and the items cover each static
 *   (cell, global 32-row block) of the reference's work list (src/s1cell.py:161-168) exactly once
 *   (index.static_chunks(off, 32, 4)).
 *   Mode 1: the item covers rows [max(prow, ps), min(prow + 128, pe)) (128 rows at most, as eight 16-row
 *   blocks from prow); the items cover each row of each cell exactly once (any grouping; prow = ps + 128 j,
 *   index.row_chunks(off, 128), is the one that wastes least). For every query q of the cell's pair list:
 *     acc = sum_j q8[q][j] * Z[n][j] (int32, exact), est = fmaf((float)acc * qs[q], zs[n], qcp[pair]).
 *   mode 0 (first pass): bm[(q*n1 + qrank[pair])*MB + blk - cs/32] = max over the block's rows in the
 *     cell; entries of blocks a cell does not have are left untouched.
 *   mode 1 (emit): every (q, n) with est >= t0[q] increments cnt[q]; the first CAP of them are stored in
 *     bval[q*CAP + idx] = est, bpos[q*CAP + idx] = n. cnt must be zero before the call.
 * R must be 256. Z must have at least max(pe) rows; N is its row count.
 */
int fvs_i8_scan(int32_t mode, int32_t P, const int8_t *q8, const float *qs, const int32_t *qid,
                const int32_t *qrank, const int32_t *coff, const int32_t *ccnt, const int32_t *pcell,
                const int32_t *prow, const int32_t *ps, const int32_t *pe, const int8_t *Z, const float *zs,
                int64_t N, int32_t R, const float *qcp, const float *t0, int32_t *cnt, float *bval,
                int32_t *bpos, float *bm, int32_t CAP, int32_t MB, int32_t n1, void *stream);

/*
 * Threshold t0 (a10). Replaces throughput/enginei8.py:53-55
 *   (v = bmc[inv]; top = v.topk(min(r, n1*MB)); t0 = min(top where top > -1e29 else 1e30)).
 *   bm f32 [B, n1, MB] written by fvs_i8_scan mode 0; probe i32 [B, npr]; off i32 [NC+1] cell offsets.
 *   Valid values of query q: bm[q][j][b] for j < n1 and b < blocks(cell probe[q][j]).
 *   t0[q] = the min(r, n1*MB, #valid)-th largest valid value, or 1e30 if none is valid.
 *   A probe id outside [0, NC) among the first n1 reads no offsets and sets t0[q] = 1e30: the query then
 *   emits nothing, and its exactness flag (K <= cnt) is cleared.
 *   cnt i32 [B] (may be NULL): set to 0, the emit pass's candidate counters (saves a fill launch).
 */
int fvs_threshold(const float *bm, const int32_t *probe, int32_t npr, const int32_t *off, int32_t NC, int64_t B,
                  int32_t n1, int32_t MB, int32_t r, float *t0, int32_t *cnt, void *stream);

/*
 * Final stage-1 selection (a12) and the delta rule (a14). Replaces throughput/enginei8.py:60
 * (t = bval.topk(K); pos = bpos[t]; ok = K <= cnt <= M) and :87-88 (ncnt).
 *   bval f32 [B, M], bpos i32 [B, M], cnt i32 [B]: the emit buffers (only the first min(cnt, M)
 *   entries of a row are read). pos i32 [B, K], est1 f32 [B, K] sorted by (est descending, pos
 *   ascending); rows with fewer than K entries are completed with (est -1e30, pos 0).
 *   ok u8 [B] = (K <= cnt <= M). ncnt i32 [B] = #{j < K : est1[j] >= est1[kd] - delta} when
 *   delta >= 0 (f32 subtraction), K otherwise. K <= 4096, 0 <= kd < K.
 */
int fvs_select(const float *bval, const int32_t *bpos, const int32_t *cnt, int64_t B, int32_t M, int32_t K,
               int32_t kd, float delta, int32_t *pos, float *est1, uint8_t *ok, int32_t *ncnt, void *stream);

/*
 * Nibble lookup tables of the uniform tiered code (a13). Replaces luts_fused/_lut_kernel
 * (throughput/s2lut.py:108-126).
 *   Zq fp16 [B, D] (the rotated queries, Qb.half() @ VP16[:, :D]); tiers i32 [T][3] = (start, end, bits)
 *   is a HOST array. L [B, D/4*16] is fp16 when half != 0, else f32:
 *     L[q][n*16 + v] = sum_{i<4} Zq[q][4n+i] * ((v >> (3-i)) & 1), as fmaf in i order from +0.
 *   qsum, qn2 f32 [T, B]: (float) of the double sums over the tier's coordinates of Zq and Zq^2, with
 *   the 64-lane order of qc (lane = offset inside the tier % 64, then the xor butterfly).
 */
int fvs_lut_build(const uint16_t *Zq, int64_t B, int32_t D, int32_t T, const int32_t *tiers, int32_t half,
                  void *L, float *qsum, float *qn2, void *stream);

/*
 * LUT stage 2 with error bars (a15). Replaces score_lut/_score_lut/_tier_lut (throughput/s2lut.py:48-106)
 * over the packed 512-byte-class records of src/tiered_fused.py:112-125.
 *   pos i32 [B, K] sorted positions; qc f32 [B]; L (fp16 if half else f32) [B, LW];
 *   qsum, qn2 f32 [T, B]; rec u8 [N, RB]: tier t plane p at toff[t] + p*(d_t/8), then (scale, sigma)
 *   fp16 pairs per tier at soff + 4t; tiers i32 [T][3], deltas f32 [T], toff i32 [T] are HOST arrays.
 *   nt: score only tiers 0 .. nt-1 (1 <= nt <= T; 0 = all T), the partial estimate of
 *   score_lut(..., nt=NT) that ranks the progressive stage's candidates (throughput/s2lut.py:92-93,
 *   throughput/enginei8.py:82-85); the record layout is still checked against all T tiers.
 *   ncnt i32 [B] or NULL (score all K). est, sd f32 [B, K]; slots m >= ncnt[q] get (-1e30, 0).
 *   Limits: LW % 128 == 0 (whole 512-byte table groups; LW = 4 d for tiers of whole 32-coordinate
 *   blocks), K <= 4096, and the record's plane and pair dwords, rounded up to 32, at most 512
 *   (FVS_E_CAPACITY otherwise: the per-dword schedule travels as a 2 KiB kernel argument).
 * Canonical arithmetic: each LUT entry is turned into the integer fx = rint(L * 2^(24-s)), with
 * s = max(0, E - 3) where max|L| of the query = f * 2^E, f in [0.5, 1) (frexp); the tier sums
 *   A_t = sum_p 2^(b-1-p) sum_j (fx[hi nibble] + fx[lo nibble]) are exact integers. Then, in f32:
 *   a = ldexpf((float)A_t, s - 24); a = delta_t * fmaf(-mid_t, qsum[t], a); est = fmaf(a, scale_t, est);
 *   var = fmaf(qn2[t] * sig_t, sig_t, var), for t = 0..nt-1, from est = qc[q], var = 0; sd = sqrtf(var)
 *   (the multiply-adds fused as the reference's compiled kernel fuses them).
 */
int fvs_lut_score(const int32_t *pos, const float *qc, const void *L, int32_t half, int32_t LW,
                  const float *qsum, const float *qn2, const uint8_t *rec, int64_t N, int32_t RB, int32_t soff,
                  int32_t T, const int32_t *tiers, const float *deltas, const int32_t *toff, int32_t nt,
                  const int32_t *ncnt, int64_t B, int32_t K, float *est, float *sd, void *stream);

/*
 * LUT stage 2 fused with its table build (a13 + a15): the same est and sd as fvs_lut_build followed by
 * fvs_lut_score with the same half, but each query's table and tier sums are formed inside the scoring
 * kernel from its rotated query (throughput/s2lut.py:108-126 feeding :48-106), so the table never goes
 * through memory and the separate build launch disappears.
 *   Zq fp16 [B, D] (as fvs_lut_build); D % 32 == 0, D <= 4096, and the last tier ends at D. The other
 *   arguments and the canonical arithmetic are fvs_lut_score's (with LW = D / 4 * 16).
 */
int fvs_lut_score_zq(const int32_t *pos, const float *qc, const uint16_t *Zq, int32_t D, int32_t half,
                     const uint8_t *rec, int64_t N, int32_t RB, int32_t soff, int32_t T, const int32_t *tiers,
                     const float *deltas, const int32_t *toff, int32_t nt, const int32_t *ncnt, int64_t B, int32_t K,
                     float *est, float *sd, void *stream);

/*
 * Error-bar classification, exact refinement and final top-k (a16, a17, a18). Replaces
 * throughput/enginei8.py:92-95, src/engine3.py:143-146 and src/stage3_zc.py:11-27.
 *   est, sd f32 [B, K]; pos i32 [B, K]; order i32 [N]; H fp16 [n_ids, d] in id order (device memory or a
 *   pinned device-mapped host buffer); Q f32 [B, d].
 *   lo = est - z*sd, hi = est + z*sd; sure = lo > (k+1)-th largest hi; amb = hi >= k-th largest lo and not sure.
 *   score = est + 10 (sure), exact <H[id], Q> (amb), -1e9 (other).
 *   ids i32 [B, K] = order[pos] (pos itself when order is NULL, for rows H stored in sorted order);
 *   I i32 [B, k] = ids of the top-k scores (score descending, slot ascending);
 *   scores f32 [B, k]: the exact score of an ambiguous pick, the estimate of a sure one;
 *   reads i32 [B] = #amb. Exact dot canonical order: lane l (0..63) sums elements 8g..8g+7 of groups
 *   g = l, l+64, ... with fmaf in element order, then acc += shfl_xor(acc, o) for o = 32, 16, 8, 4, 2, 1.
 * k < K <= 4096; d a multiple of 8.
 */
int fvs_refine(const float *est, const float *sd, const int32_t *pos, const int32_t *order, const uint16_t *H,
               const float *Q, int64_t B, int32_t K, int32_t d, float z, int32_t k, int32_t *ids, int32_t *I,
               float *scores, int32_t *reads, void *stream);

/*
 * Stage 3 split for rows outside GPU-visible memory (the NVMe row tier of the reference's Engine12,
 * src/engine3.py:204-233, which classifies on the GPU, reads the ambiguous rows with its asynchronous
 * reader and scores them). Together the two calls give the results of fvs_refine over the same rows.
 * fvs_classify: ids [B,K] (order[pos] or pos), flag u8 [B,K] (1 sure, 2 ambiguous, 0 neither, by the
 *   bounds of fvs_refine), namb [B], aslot [B,K]: the ambiguous slots in ascending slot order.
 * fvs_refine_rows: rows fp16 [sum namb, d] (device or pinned host) hold the row of ambiguous slot
 *   aslot[q][j] at roff[q] + j (roff i64 [B]); outputs I, scores, reads as fvs_refine.
 */
int fvs_classify(const float *est, const float *sd, const int32_t *pos, const int32_t *order, int64_t B, int32_t K,
                 float z, int32_t k, int32_t *ids, uint8_t *flag, int32_t *namb, int32_t *aslot, void *stream);
int fvs_refine_rows(const float *est, const uint8_t *flag, const int32_t *aslot, const int32_t *namb,
                    const int64_t *roff, const int32_t *ids, const uint16_t *rows, const float *Q, int64_t B,
                    int32_t K, int32_t d, int32_t k, int32_t *I, float *scores, int32_t *reads, void *stream);

/* ============================================================ routing-free scan (brute force)
 * The reference's routing-free stage 1 (throughput/brute.py:10-51, throughput/cbrute.py:22-64): every query's
 * int8 code against every stored code, with a sample-derived threshold. */

/*
 * int8 codes of rows (throughput/brute.py:46-47 for the stored rows, :50-52 for queries, any width R): for each
 * row r of z f32 [n, R], a = max(max_j |z[r][j]|, 1e-12f) / 127.0f and q[r][j] = clamp(rintf(z[r][j] / a),
 * -127, 127); scale[r] = a (f32) and scale16[r] = a rounded to fp16 (nearest even), each skipped when NULL.
 */
int fvs_quantize_i8(const float *z, int64_t n, int32_t R, int8_t *q, float *scale, uint16_t *scale16, void *stream);

/*
 * Fragment-tiled copy of a code matrix X i8 [n, R] (row-major), zero-padded to npad rows and Rp columns: the
 * layout fvs_dense_scan reads. The 1 KB block (rb, s) at T + (rb * Rp/32 + s) * 1024 holds, for lane
 * 32 h + li (0..63), the 16 bytes X[32 rb + li][32 s + 16 h .. + 15] (zero past row n or column R).
 * R a multiple of 16; Rp >= R a multiple of 32; npad >= n a multiple of 32; X and T 16-byte aligned.
 * T holds npad * Rp bytes.
 */
int fvs_dense_pack(const int8_t *X, int64_t n, int32_t R, int64_t npad, int32_t Rp, int8_t *T, void *stream);

/*
 * Sample threshold of the routing-free scan (throughput/brute.py:59: t0 = scores.topk(r, 1).values[:, -1]):
 * t0[q] = the r-th largest of S f32 [B, n] row q, 1 <= r <= n; cnt[q] = 0 when cnt is not NULL (the emit
 * pass's counters).
 */
int fvs_dense_threshold(const float *S, int64_t B, int32_t n, int32_t r, float *t0, int32_t *cnt, void *stream);

/*
 * Dense int8 scan on MFMA: est[q][n] = ((float)acc * qs[q]) * (float)zs[n] (two products in this order), with
 * acc = sum_j Q[q][j] * Z[n][j] exact in int32 (Qt, Zt: fvs_dense_pack layout of the query and stored codes,
 * Bpad and Npad rows). Replaces brute.py's _scan (throughput/brute.py:7-35): mode 0 writes the dense scores
 * out f32 [B, N] (its MODE 0, used on the threshold sample); mode 1 is its MODE 1: every (q, n) with
 * est >= t0[q] increments cnt[q] (zeroed by the caller) and the first CAP of a query are stored at
 * bval[q*CAP + idx] = est, bpos[q*CAP + idx] = n (in no particular order).
 *   qs f32 and (mode 1) t0 f32 hold Bpad entries, zs fp16 holds Npad entries (entries past B and N are read,
 *   never used). R (the packed width Rp) a multiple of 64; Bpad a multiple of 128; Npad a multiple of 256.
 */
int fvs_dense_scan(int32_t mode, const int8_t *Qt, const float *qs, int64_t B, int64_t Bpad, const int8_t *Zt,
                   const uint16_t *zs, int64_t N, int64_t Npad, int32_t R, const float *t0, int32_t *cnt, float *bval,
                   int32_t *bpos, int32_t CAP, float *out, void *stream);

/* ============================================================ trellis engine (latency mode)
 * The default engine of the reference (src/engine_cell.py:70-102 EngineS, src/engine3.py:135-175 Engine8):
 * cell-residual bitshift-trellis codes in stage 1 and the Lloyd-Max tiered code in stage 2. */

/*
 * Trellis encoder (a20). Replaces viterbi_fused.viterbi_paths_fused (src/viterbi_fused.py:7-46), the
 * word packing paths_to_words (src/trellis_scan.py:10-18) and the scale of cellify (src/engine_cell.py:19-22).
 *   Zs f32 [n, R] normalised residual rows (|row| = sqrt(R)); nz f32 [n] their norms; tab f32 [2^L] = alpha*T.
 *   words u32 [n, W], W = (R + L - 1 + 31) / 32: the L bits of the first state (MSB first), then the lowest
 *   bit of each later state, first bit in the most significant position of word 0.
 *   scale1 fp16 [n] = nz / (fip * |Y|), fip = <Zs, Y> / (|Y| sqrt(R)), Y = tab[path];
 *   paths i32 [n, R] or NULL.
 * Canonical order: cost_0(s) = d*d, d = Zs[0] - tab[s]; cost_j(s) = min(cost(s >> 1), cost((s >> 1) | 2^(L-1)))
 *   + d*d, the second predecessor taken only when strictly cheaper; the last state is the smallest index of
 *   minimum cost. |Y|^2 and <Zs, Y> are double sums (lane = j % 64, xor butterfly), then f32.
 * R must be 256; L in 8..10.
 */
int fvs_trellis_encode(const float *Zs, const float *nz, int64_t n, int32_t R, const float *tab, int32_t L,
                       uint32_t *words, int32_t W, uint16_t *scale1, int32_t *paths, void *stream);

/*
 * Trellis stage-1 scan (a20 decode, a21 search_static kernels _first_compact_s / _emit_loop_s,
 * src/s1cell.py:121-154; the same selection serves a22's batch sizes). Same work list, pair lists and
 * outputs as fvs_i8_scan, over the static (cell, 32-row block) items of static_blocks (not the grouped
 * chunks); qcp = (float)QM[q][c] (no norm factor).
 *   Qr f32 [B, R] = Qb @ W1; words u32 [n, W] and scale1 fp16 [n] hold index rows row0 .. row0 + n - 1 (the
 *   whole index with row0 = 0, or a staged chunk that covers every row of the P items); tab f32 [2^L].
 *   words/scale1 may be device memory or pinned, device-mapped host memory.
 *   state_j = bits j .. j+L-1 of the row's stream (MSB first), v_j = tab[state_j];
 *   est = fmaf((float)scale1, lo + hi, qcp), lo = sequential fmaf over j < R/2 of v_j * Qr[j] from +0,
 *   hi likewise over j >= R/2.
 *   half = 1: v_j and Qr[j] are each rounded to fp16 (nearest, ties to even) before the products, the operand
 *   precision of the reference's tensor-core dot in search_static / search_mask (src/s1cell.py:127,131-132,
 *   147,151-152; src/s1small_cell.py:57-59); half = 0 keeps fp32 operands, as its small-batch kernels do
 *   (src/s1small_cell.py:17-21,101). The products of fp16 operands are exact in fp32, so the accumulation
 *   order above is the only rounding left.
 * nsplit (1 .. 64): each item's queries are split into nsplit consecutive parts, one wave each (the same
 * results; for launches over few items, such as the host-resident engine's streamed chunks).
 * R must be 256; 2 <= L <= 12.
 */
int fvs_tr_scan(int32_t mode, int32_t P, const float *Qr, const int32_t *qid, const int32_t *qrank,
                const int32_t *coff, const int32_t *ccnt, const int32_t *pcell, const int32_t *pblk, const int32_t *ps,
                const int32_t *pe, const uint32_t *words, int64_t row0, int32_t W, const uint16_t *scale1, const float *tab,
                int32_t L, int32_t R, int32_t half, const float *qcp, const float *t0, int32_t *cnt, float *bval,
                int32_t *bpos, float *bm, int32_t CAP, int32_t MB, int32_t n1, int32_t nsplit, void *stream);

/*
 * The host-resident engine's streamed stage-1 pass (config 5; the reference reads the stage-1 codes
 * zero-copy, host_resident/space_x.py:17-32; here the code tiles are copied, as the configuration asks):
 * for each chunk i, one hipMemcpyAsync on `side` copies the chunk's block -- its rows' trellis words
 * (int32 [n, W]), then their fp16 scales, padded to 16 bytes -- from pinned host memory `stage_h` into
 * staging slot i % 2 (slot_bytes each), and `stream` runs fvs_tr_scan over the chunk's items once the
 * copy has landed (words, scale1 = the slot, row0 = the chunk's first row); a slot is refilled only after
 * the scan that read it, and the first copies wait for the work already queued on `stream`.
 * chunks: HOST int64 [nchunks][5] = (first row, end row, first item, end item, byte offset of the block in
 * stage_h). The other arguments are fvs_tr_scan's, with the work list (pcell, pblk, ps, pe) of the whole
 * index. The ordering events are created once per device and reused: calls on one device must not overlap.
 */
int fvs_tr_scan_streamed(int32_t mode, int32_t nchunks, const int64_t *chunks, const uint8_t *stage_h,
                         uint8_t *slot0, uint8_t *slot1, int64_t slot_bytes, void *side, const float *Qr,
                         const int32_t *qid, const int32_t *qrank, const int32_t *coff, const int32_t *ccnt,
                         const int32_t *pcell, const int32_t *pblk, const int32_t *ps, const int32_t *pe, int32_t W,
                         const float *tab, int32_t L, int32_t R, int32_t half, const float *qcp, const float *t0,
                         int32_t *cnt, float *bval, int32_t *bpos, float *bm, int32_t CAP, int32_t MB, int32_t n1,
                         int32_t nsplit, void *stream);

/*
 * Routing on fp32 keys (a7 for the default engine). Replaces route() (src/engine_cell.py:40-42):
 * (QM.float() * inv_mnorm).topk(nprobe). QM fp16 [B, NC]; scale f32 [NC]; probe i32 [B, nprobe] sorted by
 * (key descending, cell ascending), key = (float)QM[q][c] * scale[c], or ((float)QM[q][c] + qadd[q]) * scale[c]
 * when qadd (f32 [B]) is given (host_resident/space_x.py:33-39). NC <= 8192, nprobe <= 4096.
 */
int fvs_route_topk_scaled(const uint16_t *QM, const float *scale, const float *qadd, int64_t B, int32_t NC,
                          int32_t nprobe, int32_t *probe, void *stream);

/*
 * fp16 routing keys of EngineI8's routing variants (throughput/enginei8.py:72-76):
 * out[q][c] = fp16(((float)QM[q][c] + qadd[q]) * scale[c]) (nearest, ties to even), where the add is left out
 * when qadd is NULL and the product when scale is NULL. ROUTE16 without NROUTE: scale = inv_mnorm, qadd = NULL
 * ((QM.float() * inv_mnorm).half()); PROJ: scale = NULL, qadd = QC ((QC[:, None] + P.float()).half()).
 * QM, out fp16 [B, NC]; scale f32 [NC]; qadd f32 [B].
 */
int fvs_route_keys(const uint16_t *QM, const float *scale, const float *qadd, int64_t B, int32_t NC, uint16_t *out,
                   void *stream);

/*
 * Lloyd-Max tiered stage 2 (a23). Replaces tiered_fused.score / _tiered_score_rec (src/tiered_fused.py:47-141).
 *   pos i32 [B, K]; qc f32 [B] = <q, c>; Zq f32 [B, D] = Qb @ VP (fp32); rec u8 [N, RB] packed records;
 *   tiers i32 [T][3] (start, end, bits) and toff i32 [T] are HOST arrays; cb f32 [T, 256]: tier t's levels
 *   in code order; ncnt i32 [B] or NULL. est, sd f32 [B, K]; slots m >= ncnt[q] get (-1e30, 0).
 * Canonical order: code_k from the tier's planes (MSB plane first); lane l (0..63) sums
 *   fmaf(cb[t][code_k], Zq[start_t + k], .) over k = l, l + 64, ... from +0, then the xor butterfly gives
 *   a_t; est = fmaf(a_t, scale_t, est), var = fmaf(qn2_t * sig_t, sig_t, var) for t = 0..T-1 from
 *   est = qc, var = 0; sd = sqrtf(var); qn2_t = (float) double sum of Zq^2 over the tier (lane tree).
 */
int fvs_tiered_score(const int32_t *pos, const float *qc, const float *Zq, int32_t D, const uint8_t *rec, int64_t N,
                     int32_t RB, int32_t soff, int32_t T, const int32_t *tiers, const int32_t *toff, const float *cb,
                     const int32_t *ncnt, int64_t B, int32_t K, float *est, float *sd, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* FVS_H */
