/*
 * ringmaster_amd — C ABI of the MI355X (gfx950) ring-attention compute path.
 *
 * Every entry point:
 *   - takes plain device pointers, element strides and sizes (no torch types);
 *   - validates its arguments on the host before any launch and returns 0 on
 *     success or a negative RMX_E* code (the message is in rmx_last_error());
 *   - never throws, aborts or frees across the ABI; all memory is owned by the
 *     caller;
 *   - launches asynchronously on the caller's HIP stream (a hipStream_t passed
 *     as void*; NULL is the default stream);
 *   - keeps no mutable global state apart from the per-thread error string (and the
 *     per-device address of the one allocation-free entry point's scratch array).
 *
 * Tensor conventions follow the reference ring path: q/k/v/out are
 * [batch, seq, heads, dim] with arbitrary element strides for the first three
 * axes and a contiguous last axis; lse is [batch, heads, seq] fp32 (natural
 * log) with a contiguous seq axis. bf16 tensors are passed as uint16_t bit
 * patterns.
 */
#ifndef RINGMASTER_AMD_H
#define RINGMASTER_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RMX_ABI_VERSION 18 /* 3: Mamba2 correction bwd; 4: nlse; 5: CP conv1d; 6: dt cumsum;
                              7: effective dt in/out of the dt cumsum, shard final state;
                              8: allocation-free Mamba2 correction bwd;
                              9: carried-in state h_in / dh_in of the linear scan;
                              10: L-parallel linear scan (workspace argument);
                              11: sliding windows, attention head_dim any multiple of 8
                                  up to 128; 12: fp16 attention (layout dtype);
                              13: attention dropout;
                              14: workspace of the Mamba2 shard-state backward;
                              15: attention head_dim up to 256;
                              16: per-batch-row document metadata (layout m_sb),
                                  dropout with document masks;
                              17: rmx_linear_scan_status;
                              18: right-bounded windows (problem window_right) */

/* error codes */
#define RMX_OK 0
#define RMX_EINVAL (-1)   /* bad argument: maps to ValueError */
#define RMX_EUNSUPPORTED (-2) /* valid but not implemented here: NotImplementedError */
#define RMX_EDEVICE (-3)  /* HIP runtime / launch failure: RuntimeError */

/* 16-bit element types of q, k, v, out, dout and the 16-bit gradients of one attention call */
#define RMX_DTYPE_BF16 0
#define RMX_DTYPE_F16 1

/* block mask kinds (ring/kernels.py:64-67, ring/varlen_blocks.py:51-58) */
#define RMX_MASK_FULL 0   /* every (q, k) pair attends */
#define RMX_MASK_CAUSAL 1 /* bottom-right aligned causal: k <= q + (sk - sq) + window_right
                             (window_right = 0: causal attention) */
#define RMX_MASK_DOC 2    /* q_doc[q] == k_doc[k] && k_gidx[k] <= q_gidx[q]; the four arrays
                             advance by the layout's m_sb per batch row */
/* RMX_DROPOUT: with dropout_p > 0, element (b, h, q, k) of a problem (h the q head) is kept when
 *   fmix32(bhmix ^ (q + drop_q0) * 0x85ebca77 ^ (k + drop_k0) * 0xc2b2ae3d) >= floor(p * 2^32),
 *   bhmix = fmix32(drop_seed_lo ^ fmix32(drop_seed_hi ^ (b * hq + h) * 0x9e3779b9)),
 * all arithmetic mod 2^32, fmix32 the MurmurHash3 32-bit finalizer, p the float dropout_p
 * (floor of its exact value times 2^32); kept probabilities are scaled by 1 / (1 - p) and lse
 * is the undropped one (the Dao flash-attention semantics).
 * The backward must get the forward's layout seed and each problem's drop_q0 / drop_k0. */
/* A problem's sliding window (has_window = 1) masks every pair further apart than
 * window_left: pos_q - pos_k > window_left, with the bottom-right aligned positions
 * pos_q = q + (sk - sq), pos_k = k (ring/kernels.py:68-72), or the global indices
 * q_gidx / k_gidx under RMX_MASK_DOC (ring/loop.py:185-186). It applies on top of the
 * mask kind; window_left may be any int32 (a negative bound also masks the diagonal,
 * which is how one block of a windowed ring sees the window of the global sequence).
 * Rows left with no key get lse = -inf and out = 0, as with document masks.
 * A window bounded on the right as well (flash attention's window_size = (left, right),
 * right >= 0, on a non-causal block: pos_k - pos_q > right masked) runs as RMX_MASK_CAUSAL
 * with window_right = right; window_right must be 0 under the other mask kinds. */

/* forward epilogue modes (online-softmax merge, ring/merge.py:20-31) */
#define RMX_FWD_WRITE 0       /* out/lse := this block's (out, lse); acc_out (nullable)
                                 := the same out in fp32 */
#define RMX_FWD_ACC_INIT 1    /* acc_out/acc_lse := this block (first ring step) */
#define RMX_FWD_ACC_MERGE 2   /* acc := merge(acc, block) */
#define RMX_FWD_ACC_FINAL 3   /* out(bf16)/lse := merge(acc, block); acc_out := the merged
                                 out in fp32; acc_lse untouched */

/* backward gradient output modes */
#define RMX_GRAD_WRITE_BF16 0 /* grad_bf16 := this block's gradient */
#define RMX_GRAD_WRITE_F32 1  /* grad_acc := this block's gradient */
#define RMX_GRAD_ACC_F32 2    /* grad_acc += this block's gradient */
#define RMX_GRAD_ACC_FINAL 3  /* grad_bf16 := grad_acc + this block's gradient */
#define RMX_GRAD_NONE 4       /* this gradient is not computed (its kernel is not launched
                                 when no problem of the call asks for it) */

#define RMX_MAX_BATCHED 16    /* problems per launch; more are split by the library */

/* Layout shared by every problem of one batched attention call. */
typedef struct rmx_attn_layout {
  int32_t batch, hq, hkv;           /* hq % hkv == 0 (GQA: kv_head = q_head / (hq/hkv)) */
  int32_t head_dim;                 /* a multiple of 8, at most 256: the kernels compute at 64,
                                       128 or 256 and read the columns past head_dim as zeros */
  float scale;                      /* softmax scale (1/sqrt(head_dim) by default) */
  int32_t mask;                     /* RMX_MASK_* */
  int32_t dtype;                    /* RMX_DTYPE_*: the 16-bit tensors ("bf16" below) hold this
                                       type; accumulators, lse and delta stay fp32 */
  float dropout_p;                  /* attention dropout probability in [0, 1); 0: none. The
                                       mask is a hash of (drop_seed, batch, q head, query, key),
                                       see RMX_DROPOUT below */
  uint32_t drop_seed_lo, drop_seed_hi;
  /* element strides (batch, seq, head) */
  int64_t q_sb, q_ss, q_sh;
  int64_t k_sb, k_ss, k_sh;
  int64_t v_sb, v_ss, v_sh;
  int64_t o_sb, o_ss, o_sh;   /* bf16 out, dout and the bf16 gradient of q */
  int64_t a_sb, a_ss, a_sh;   /* fp32 running out / fp32 dq accumulator */
  int64_t l_sb, l_sh;         /* lse, acc_lse, delta: [batch, head, seq], seq stride 1 */
  int64_t dk_sb, dk_ss, dk_sh; /* bf16 dk/dv outputs */
  int64_t ka_sb, ka_ss, ka_sh; /* fp32 dk/dv accumulators */
  int64_t m_sb;               /* RMX_MASK_DOC: int32 element stride between the batch rows of
                                 q_gidx, k_gidx, q_doc and k_doc (0: every row shares them;
                                 ring/loop.py:178 gives each packed row its own documents) */
} rmx_attn_layout;

/* One block-attention forward problem: q[sq] attends k/v[sk]. */
typedef struct rmx_fwd_problem {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* out;        /* bf16, may be NULL in ACC_INIT/ACC_MERGE */
  float* lse;           /* fp32 [b, hq, sq], may be NULL in ACC_INIT/ACC_MERGE */
  float* acc_out;       /* fp32 running out (ACC_* modes) */
  float* acc_lse;       /* fp32 running lse (ACC_* modes) */
  const int32_t* q_gidx; /* RMX_MASK_DOC: global token index of each q row (non-decreasing) */
  const int32_t* k_gidx; /* RMX_MASK_DOC: global token index of each k row (non-decreasing).
                            The kernels only compare it with q_gidx (k_gidx <= q_gidx, and the
                            window on q_gidx - k_gidx): a caller that passes each key's document
                            start instead gets same-document attention without the causal
                            bound (the non-causal packed ring, ring/loop.py:149,183-184) */
  const int32_t* q_doc;  /* RMX_MASK_DOC: document id of each q row (non-decreasing), i.e.
                            doc_ids_from_cu(cu_seqlens)[q_gidx] (ring/varlen_blocks.py:45-48) */
  const int32_t* k_doc;  /* RMX_MASK_DOC: document id of each k row (non-decreasing) */
  int32_t sq, sk;
  int32_t mode;          /* RMX_FWD_* */
  int32_t has_window;    /* 0: no window; 1: window_left bounds pos_q - pos_k (see above) */
  int32_t window_left;
  int32_t drop_q0, drop_k0; /* dropout coordinates of the first query / key (RMX_DROPOUT) */
  int32_t window_right;  /* RMX_MASK_CAUSAL: pos_k - pos_q <= window_right, 0 <= window_right
                            <= 2^28 (0: causal); 0 under the other mask kinds */
} rmx_fwd_problem;

/* One block-attention backward problem, using the GLOBAL (merged) out/lse. */
typedef struct rmx_bwd_problem {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* dout;  /* bf16, o_* strides */
  const float* lse;      /* fp32 [b, hq, sq] global lse */
  const float* delta;    /* fp32 [b, hq, sq] rowsum(dout * out_global) */
  const float* nlse;     /* fp32 [b, hq, sq] -lse * log2(e), written by rmx_attn_bwd_delta;
                            required when dkv_mode != RMX_GRAD_NONE */
  float* dq_acc;         /* fp32, a_* strides (F32 modes) */
  uint16_t* dq;          /* bf16, o_* strides (WRITE_BF16 / ACC_FINAL) */
  float* dk_acc;         /* fp32, ka_* strides */
  float* dv_acc;
  uint16_t* dk;          /* bf16, dk_* strides */
  uint16_t* dv;
  const int32_t* q_gidx; /* RMX_MASK_DOC: as in rmx_fwd_problem */
  const int32_t* k_gidx;
  const int32_t* q_doc;
  const int32_t* k_doc;
  int32_t sq, sk;
  int32_t dq_mode;       /* RMX_GRAD_* */
  int32_t dkv_mode;      /* RMX_GRAD_* */
  int32_t has_window;    /* as in rmx_fwd_problem: the forward's window of the same block */
  int32_t window_left;
  int32_t drop_q0, drop_k0; /* as in rmx_fwd_problem: the forward's dropout coordinates */
  int32_t window_right;  /* as in rmx_fwd_problem: the forward's right bound */
} rmx_bwd_problem;

int32_t rmx_abi_version(void);
const char* rmx_last_error(void);

/*
 * Batched block-attention forward: softmax(scale*Q K^T + mask) V and its fp32
 * LSE for each problem, with the online-softmax merge into a running fp32
 * (out, lse) fused into the epilogue.
 * Replaces the Dao `_flash_attn_forward` op the zigzag ring calls
 * (ring/zigzag.py:131,134,138 via ring/p2p_attn.py:27-62) together with the
 * `_merge_full`/`_merge_slice` that follows it (ring/zigzag.py:49-67), and
 * backs the block provider contract of ring/kernels.py:28-85.
 */
int32_t rmx_attn_fwd(const rmx_attn_layout* layout, const rmx_fwd_problem* problems,
                     int32_t nproblems, void* stream);

/*
 * delta[b, h, s] = sum_d dout * out (FlashAttention-2 backward preprocess;
 * the rowsum(dO * O) of ring/p2p_attn.py:243-281). `out` is bf16 with the o_*
 * strides (out_is_f32 == 0, what a Dao-style bwd receives) or the fp32 final
 * out left in acc_out by the forward, with the a_* strides (out_is_f32 != 0):
 * the fp32 form matches the reference `math` provider, whose autograd never
 * rounds out to bf16. dout uses the o_* strides.
 * When nlse is not NULL, the same pass also writes nlse[b, h, s] = -lse * log2(e)
 * from the global lse (the exponent offset the dK/dV kernel adds per query);
 * lse, delta and nlse share the l_* strides.
 */
int32_t rmx_attn_bwd_delta(const rmx_attn_layout* layout, const void* out, int32_t out_is_f32,
                           const uint16_t* dout, float* delta, const float* lse, float* nlse,
                           int32_t sq, void* stream);

/*
 * Batched block-attention backward with the global out/lse (ring identity,
 * ring/p2p_attn.py:243-281): dQ, dK, dV of each problem, GQA folded over the
 * q-head group. Replaces the Dao `_flash_attn_backward` calls of
 * ring/zigzag.py:219,230,239 and the bf16 `+=` accumulations around them.
 * Problems of one call must not write the same dk/dv rows (a ring step visits
 * each KV block once).
 */
int32_t rmx_attn_bwd(const rmx_attn_layout* layout, const rmx_bwd_problem* problems,
                     int32_t nproblems, void* stream);

/*
 * Standalone online-softmax merge, `update_out_and_lse` (ring/merge.py:20-31):
 *   new = logaddexp(lse, blk_lse); out = e^(lse-new) out + e^(blk_lse-new) blk_out.
 * out: fp32 [b, s, h, d] (strides o_*), lse: fp32 [b, s, h] (strides l_*),
 * blk_out: [b, s, h, d] (strides bo_*) of type blk_type, RMX_BLK_BF16 (0), RMX_BLK_F32 (1)
 * or RMX_BLK_F16 (2),
 * blk_lse: fp32 [b, h, s] (strides bl_*). init != 0: out/lse := block
 * (the `out is None` branch, ring/merge.py:27-28). Updated in place.
 */
#define RMX_BLK_BF16 0
#define RMX_BLK_F32 1
#define RMX_BLK_F16 2
int32_t rmx_lse_merge(float* out, float* lse, const void* blk_out, int32_t blk_type,
                      const float* blk_lse, int32_t batch, int32_t seq, int32_t heads,
                      int32_t head_dim, const int64_t* o_strides /*3*/,
                      const int64_t* l_strides /*3*/, const int64_t* bo_strides /*3*/,
                      const int64_t* bl_strides /*2: batch, head*/, int32_t init,
                      void* stream);

/*
 * Zigzag (head_tail) shard of `batch` rows of `seq` tokens over `world` ranks:
 * rank r receives chunks r and 2*world-1-r of the sequence padded to a multiple
 * of 2*world (balancers.py:18-29, shard.py:150-176), early chunk first. Each
 * token is a row of row_bytes bytes; src is [batch, seq, row] with batch stride
 * src_bstride bytes. rank < 0: dst is [world, batch, local, row] (every shard);
 * rank >= 0: dst is [batch, local, row] (that rank's shard only). Rows past
 * `seq` (the padding) are copied from pad_row, a device row of row_bytes bytes,
 * or zero-filled when pad_row is NULL (shard.py:130-147).
 */
int32_t rmx_zigzag_gather(const void* src, void* dst, int32_t batch, int32_t seq,
                          int32_t world, int32_t rank, int64_t row_bytes, int64_t src_bstride,
                          const void* pad_row, void* stream);

/* Inverse of rmx_zigzag_gather for rank < 0: dst[batch, seq, row] (batch stride
 * dst_bstride bytes) from the [world, batch, local, row] shards, the unshard of
 * tests/test_zigzag_shard.py:39-43; padding rows are dropped. */
int32_t rmx_zigzag_scatter(const void* src, void* dst, int32_t batch, int32_t seq,
                           int32_t world, int64_t row_bytes, int64_t dst_bstride,
                           void* stream);

/*
 * Context-parallel linear scan h_t = a_t h_{t-1} + b_t (strategies/state_passing.py:19-59).
 * Replaces `cp_linear_scan(a, b, group)` (strategies/state_passing.py:29): with world == 1
 * and h_in it is one rank's call on its local chunk (the local zero-init scan corrected by
 * cumA * H_in, :59, where H_in is the rank-ordered prefix of the earlier ranks' (A_j, B_j),
 * :55-57); with world > 1 the sequence is `world` contiguous shards emulated in one launch
 * (each shard scans from zero, the shards' (decay, carry) pairs are prefix-combined in rank
 * order and the correction applied), starting from h_in.
 * a: fp32 [batch, L, groups] with `groups` dividing d (a[b,t,g] applies to the
 * d/groups consecutive channels of group g; groups == d is elementwise);
 * b, h: fp32 [batch, L, d] contiguous. h_in (nullable: zero): fp32 [batch, d], the state
 * before token 0. chunk_state (nullable): fp32 [world, batch, 2, d] receives each
 * shard's (A_r broadcast, B_r), what a rank contributes to the all-gather of :49-52.
 */
int32_t rmx_linear_scan_fwd(const float* a, const float* b, const float* h_in, float* h,
                            float* chunk_state, int32_t batch, int32_t L, int32_t d,
                            int32_t groups, int32_t world, void* workspace,
                            size_t workspace_bytes, void* stream);

/*
 * Workspace of the L-parallel scan path of rmx_linear_scan_fwd / _bwd for this shape (same
 * value for both directions), and through chunk_tokens (nullable) its chunk length. With
 * workspace == NULL the scan entry points run a thread per channel along the whole sequence
 * (the fast form when batch * d fills the GPU); with a workspace of at least this size they
 * run the chained scan that is parallel over L (long sequences, few channels). Only one call
 * may use a workspace at a time. With chunk_state, the L-parallel path needs L / world to
 * be a multiple of the chunk length.
 */
size_t rmx_linear_scan_workspace(int32_t batch, int32_t L, int32_t d, int32_t groups,
                                 int32_t* chunk_tokens);

/*
 * Status of the last rmx_linear_scan_fwd / _bwd call that used this workspace: synchronizes
 * the stream, then returns RMX_EDEVICE when a chunk of the L-parallel scan gave up waiting
 * for its predecessor's state (after about 0.3 s of polls; its carried state and the
 * outputs after it are NaN), RMX_OK otherwise (and for a NULL workspace). No reference
 * counterpart: the reference's sequential loop cannot stall.
 */
int32_t rmx_linear_scan_status(const void* workspace, size_t workspace_bytes, void* stream);

/*
 * Gradient of rmx_linear_scan_fwd (what autograd through the reference's loop, cumprod
 * and the all-gather's all-reduce backward computes): given dh, the forward's h and h_in
 * (nullable), writes db [batch, L, d], ADDS da [batch, L, groups] (caller zero-fills da)
 * and, when dh_in is not NULL, writes dh_in [batch, d] = a_0 * g_0, the gradient of h_in
 * (zero when L == 0), which a rank sends back to the ranks whose states formed its H_in.
 */
int32_t rmx_linear_scan_bwd(const float* a, const float* h, const float* h_in, const float* dh,
                            float* da, float* db, float* dh_in, int32_t batch, int32_t L,
                            int32_t d, int32_t groups, int32_t world, void* workspace,
                            size_t workspace_bytes, void* stream);

/*
 * Mamba2 context-parallel output correction (strategies/mamba.py:101-139):
 *   y[b,t,h,:] = out[b,t,h,:] + bf16(e^{cum_A[b,t,h]} sum_n C[b,t,g(h),n] h_prev[b,h,:,n])
 *   h_final_out[b,h] = h_final[b,h] + e^{cum_A[b,T-1,h]} h_prev[b,h]
 * with g(h) = h / (nheads / ngroups). seq_idx (nullable, int32 [batch, T]): tokens
 * with seq_idx != 0 get no correction, and no state is updated when the last
 * token of any batch row has seq_idx != 0 (h_final_out := h_final; the reference
 * tests seq_idx[:, -1].any() over the batch). Layouts (contiguous):
 * out, y: bf16 [batch, T, nheads * head_dim] (y may alias out); C: bf16
 * [batch, T, ngroups, d_state]; cum_A: fp32 [batch, T, nheads]; h_prev, h_final,
 * h_final_out: fp32 [batch, nheads, head_dim, d_state] (h_final_out may alias
 * h_final). head_dim in {32, 64, 128}; d_state in {16, 32, 64, 128, 256} with
 * head_dim * d_state <= 32768.
 */
int32_t rmx_mamba2_cp_correction(const uint16_t* out, uint16_t* y, const float* h_final,
                                 float* h_final_out, const uint16_t* C, const float* cum_A,
                                 const float* h_prev, const int32_t* seq_idx, int32_t batch,
                                 int32_t T, int32_t nheads, int32_t head_dim, int32_t ngroups,
                                 int32_t d_state, void* stream);

/*
 * Backward of rmx_mamba2_cp_correction: the gradients autograd takes through the
 * reference's torch ops (strategies/mamba.py:116-137) for C, cum_A and h_prev.
 * (The gradients of out and h_final are the upstream ones, unchanged.) Inputs:
 * gy bf16 [batch, T, nheads * head_dim] (dL/dy); ghf fp32 like h_prev
 * (dL/dh_final_out, nullable: no gradient reaches it); C, cum_A, h_prev, seq_idx
 * as in the forward. Outputs: gC bf16 like C, g_cumA fp32 like cum_A, g_hprev
 * fp32 like h_prev. workspace: device memory of at least
 * rmx_mamba2_cp_correction_bwd_workspace(...) bytes (block partials of dL/dh_prev,
 * h_prev^T split into three bf16 parts, e^{cum_A} transposed); its contents on entry
 * do not matter. head_dim in {64, 128}; d_state in {64, 128}; the head slices
 * of 64 channels come in fours from one C group ((nheads / ngroups) divisible by
 * 4 at head_dim 64, by 2 at head_dim 128); otherwise RMX_EUNSUPPORTED.
 */
size_t rmx_mamba2_cp_correction_bwd_workspace(int32_t batch, int32_t T, int32_t nheads,
                                              int32_t head_dim, int32_t ngroups, int32_t d_state);
int32_t rmx_mamba2_cp_correction_bwd(const uint16_t* gy, const float* ghf, const uint16_t* C,
                                     const float* cum_A, const float* h_prev,
                                     const int32_t* seq_idx, uint16_t* gC, float* g_cumA,
                                     float* g_hprev, void* workspace, size_t workspace_bytes,
                                     int32_t batch, int32_t T, int32_t nheads, int32_t head_dim,
                                     int32_t ngroups, int32_t d_state, void* stream);

/*
 * Allocation-free variant of rmx_mamba2_cp_correction_bwd. It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same arguments and
 * results as rmx_mamba2_cp_correction_bwd without the workspace: the workspace is a
 * file-scope device array of RMX_MAMBA2_BWD_SCRATCH_MAX bytes (96 MiB), which the library
 * holds on every GPU it runs on until the process ends. A shape whose
 * rmx_mamba2_cp_correction_bwd_workspace exceeds that maximum returns RMX_EINVAL before
 * anything is launched. The call allocates and frees nothing. Every call on one GPU
 * shares that GPU's array and its contents (none of which needs to start at zero), so
 * calls that overlap on one GPU (from other streams or threads) race. The array's
 * device address is looked up once per device, on the first call with that device
 * current; the stream must belong to the current device (RMX_EINVAL otherwise).
 */
#define RMX_MAMBA2_BWD_SCRATCH_MAX ((size_t)96 << 20)
int32_t rmx_mamba2_cp_correction_bwd_noalloc(const uint16_t* gy, const float* ghf,
                                             const uint16_t* C, const float* cum_A,
                                             const float* h_prev, const int32_t* seq_idx,
                                             uint16_t* gC, float* g_cumA, float* g_hprev,
                                             int32_t batch, int32_t T, int32_t nheads,
                                             int32_t head_dim, int32_t ngroups, int32_t d_state,
                                             void* stream);

/*
 * Mamba2 CP chunk decay from dt, the first step of the reference's CP scan
 * wrapper (strategies/mamba.py:276-283): per row (rank shard x batch) and head,
 *   e_t = softplus(dt_t + dt_bias) if dt_softplus else dt_t   (torch softplus,
 *         threshold 20; dt_bias only with dt_softplus, as in the reference)
 *   cum_A[r,t,h] = sum_{s<=t} A[h] e_s,   decay[r,h] = exp(cum_A[r,T-1,h])
 * computed in fp32. dt: [rows, T, nheads] bf16 (dt_is_f32 = 0) or fp32;
 * dt_bias, A: fp32 [nheads] (dt_bias nullable); cum_A fp32 [rows, T, nheads];
 * e (nullable): the effective dt e_t, fp32 [rows, T, nheads] (what the shard
 * state below weighs tokens with); decay fp32 [rows, nheads]; all contiguous.
 */
int32_t rmx_mamba2_dt_cumsum(const void* dt, int32_t dt_is_f32, const float* dt_bias,
                             const float* A, int32_t dt_softplus, float* cum_A, float* e,
                             float* decay, int32_t rows, int32_t T, int32_t nheads, void* stream);

/*
 * Gradient of rmx_mamba2_dt_cumsum: given dL/dcum_A (nullable), dL/de (nullable,
 * a direct gradient of the effective dt) and dL/ddecay (nullable, with the
 * forward's decay), writes dL/ddt (fp32 [rows, T, nheads]) and ADDS dL/dA and
 * dL/ddt_bias (fp32 [nheads]; dt_bias gradient only with dt_softplus; nullable)
 * (caller zero-fills them).
 */
int32_t rmx_mamba2_dt_cumsum_bwd(const void* dt, int32_t dt_is_f32, const float* dt_bias,
                                 const float* A, int32_t dt_softplus, const float* g_cum_A,
                                 const float* g_e, const float* g_decay, const float* decay,
                                 float* g_dt, float* g_A, float* g_dt_bias, int32_t rows,
                                 int32_t T, int32_t nheads, void* stream);

/*
 * Mamba2 shard final state from x, B and dt: the final_states of mamba-ssm's
 * mamba_chunk_scan_combined(..., return_final_states=True) from a zero state,
 * which the reference's CP scan wrapper gathers across ranks (mamba.py:113-141,
 * 160-172: `final` of each shard, the last document's state when packed;
 * strategies/mamba.py:250-300). Per row and head h of group g = h / (H / G):
 *   state[r,h] = sum_{t0[r] <= t < T} exp(cum_A[r,T-1,h] - cum_A[r,t,h]) e[r,t,h]
 *                x[r,t,h,:] (x) B[r,t,g,:]
 * (the SSD recurrence h_t = exp(A e_t) h_{t-1} + e_t x_t (x) B_t unrolled; the
 * weighted x is rounded to bf16 before the MFMA, sums fp32).
 * x bf16 [rows, T, H, head_dim]; B bf16 [rows, T, G, d_state]; e, cum_A fp32
 * [rows, T, H] (from rmx_mamba2_dt_cumsum); t0 int32 [rows] (nullable: 0), the
 * first token of each row's last document; state fp32 [rows, H, head_dim,
 * d_state]. head_dim and d_state in {64, 128}; contiguous, 16-byte aligned.
 */
int32_t rmx_mamba2_chunk_state(const uint16_t* x, const uint16_t* B, const float* e,
                               const float* cum_A, const int32_t* t0, float* state, int32_t rows,
                               int32_t T, int32_t nheads, int32_t head_dim, int32_t ngroups,
                               int32_t d_state, void* stream);

/*
 * Gradient of rmx_mamba2_chunk_state given g_state = dL/dstate (fp32, like
 * state): writes g_x (bf16, like x), g_B (bf16, like B), g_e and g_cum_A (fp32
 * [rows, T, H]). g_cum_A[r, T-1, h] is left as -g_w w of that token; the full
 * entry is sum_{t<T-1} g_w w = -sum_{t<T-1} g_cum_A[r, t, h], which the caller
 * writes (every weight depends on cum_A at T-1). workspace (nullable) of at least
 * rmx_mamba2_chunk_state_bwd_workspace(...) bytes, 16-byte aligned: with it (and a
 * nonzero size: head_dim 64), g_state is first converted to bf16 there and the kernel moves two
 * heads per step, reading G by LDS DMA; without it the one-head form runs. Both give
 * the same results up to fp32 summation order.
 */
size_t rmx_mamba2_chunk_state_bwd_workspace(int32_t rows, int32_t nheads, int32_t head_dim,
                                            int32_t d_state);
int32_t rmx_mamba2_chunk_state_bwd(const uint16_t* x, const uint16_t* B, const float* e,
                                   const float* cum_A, const int32_t* t0, const float* g_state,
                                   uint16_t* g_x, uint16_t* g_B, float* g_e, float* g_cum_A,
                                   int32_t rows, int32_t T, int32_t nheads, int32_t head_dim,
                                   int32_t ngroups, int32_t d_state, void* workspace,
                                   size_t workspace_bytes, void* stream);

/*
 * Mamba2 context-parallel causal conv1d with the halo (mamba.py:46-101, the conv
 * hook of the reference's Mamba2 adapter): the depthwise causal conv of every
 * rank's shard, where shard r's first width-1 outputs read the last width-1
 * tokens of shard r-1 (the all-gathered halo; zeros for r = 0). doc (nullable,
 * int32 [batch, world * local_len], doc_ids_from_cu(cu_seqlens)): taps from
 * another document contribute zero (the reference's per-document segments and
 * halo mask). y[g] = act(bias + sum_i w[i] x[g - (width-1) + i]) with
 * causal_conv1d_fn's semantics; activation 0 = none, 1 = silu.
 * x, y: bf16 [world, batch, channels, local_len] (each shard channels-first, the
 * layout causal_conv1d_fn takes), contiguous, 16-byte aligned; weight bf16
 * [channels, width]; bias bf16 [channels] (nullable). local_len % 8 == 0,
 * 1 <= width <= 9.
 */
int32_t rmx_causal_conv1d_cp(const uint16_t* x, const uint16_t* weight, const uint16_t* bias,
                             const int32_t* doc, uint16_t* y, int32_t world, int32_t batch,
                             int32_t channels, int32_t local_len, int32_t width,
                             int32_t activation, void* stream);

/*
 * Backward of rmx_causal_conv1d_cp (what autograd through the reference's halo
 * all-gather and per-shard convolutions computes): writes dx (bf16, like x; the
 * halo's gradient lands on the previous shard's last tokens) and ADDS the fp32
 * dweight [channels, width] and dbias [channels] (nullable) sums (caller
 * zero-fills them).
 */
int32_t rmx_causal_conv1d_cp_bwd(const uint16_t* x, const uint16_t* weight, const uint16_t* bias,
                                 const int32_t* doc, const uint16_t* dy, uint16_t* dx,
                                 float* dweight, float* dbias, int32_t world, int32_t batch,
                                 int32_t channels, int32_t local_len, int32_t width,
                                 int32_t activation, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RINGMASTER_AMD_H */
