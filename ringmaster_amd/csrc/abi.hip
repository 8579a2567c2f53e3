// extern "C" entry points of libringmaster_amd.so (declared in
// include/ringmaster_amd.h). Every argument is validated here, on the host,
// before anything is launched; errors are reported as negative codes with a
// per-thread message and nothing ever throws across the ABI.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "rmx_kernels.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int dev_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return RMX_OK;
  return fail(RMX_EDEVICE, "%s: %s", what, hipGetErrorString(e));
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

int check_layout(const rmx_attn_layout* L) {
  if (!L) return fail(RMX_EINVAL, "layout is NULL");
  if (L->batch < 0 || L->hq <= 0 || L->hkv <= 0)
    return fail(RMX_EINVAL, "batch/heads must be positive (batch=%d hq=%d hkv=%d)", L->batch, L->hq,
                L->hkv);
  if (L->hq % L->hkv)
    return fail(RMX_EINVAL, "Query heads must be divisible by KV heads (hq=%d hkv=%d)", L->hq,
                L->hkv);
  if (L->head_dim <= 0 || L->head_dim > 256 || L->head_dim % 8)
    return fail(RMX_EUNSUPPORTED, "head_dim %d is not supported (a multiple of 8, at most 256)",
                L->head_dim);
  if (!(L->scale > 0.f) || !std::isfinite(L->scale))
    return fail(RMX_EINVAL, "softmax scale must be finite and positive (got %g)", (double)L->scale);
  if (L->mask < RMX_MASK_FULL || L->mask > RMX_MASK_DOC)
    return fail(RMX_EINVAL, "unknown mask kind %d", L->mask);
  if (L->dtype != RMX_DTYPE_BF16 && L->dtype != RMX_DTYPE_F16)
    return fail(RMX_EINVAL, "unknown element type %d", L->dtype);
  if (!(L->dropout_p >= 0.f && L->dropout_p < 1.f))
    return fail(RMX_EINVAL, "dropout_p must lie in [0, 1) (got %g)", (double)L->dropout_p);
  if (L->m_sb < 0) return fail(RMX_EINVAL, "m_sb must be non-negative (got %lld)", (long long)L->m_sb);
  const int64_t bf[] = {L->q_sb, L->q_ss, L->q_sh, L->k_sb, L->k_ss, L->k_sh,
                        L->v_sb, L->v_ss, L->v_sh, L->o_sb, L->o_ss, L->o_sh,
                        L->dk_sb, L->dk_ss, L->dk_sh};
  for (int64_t s : bf)
    if (s < 0 || s % 8)
      return fail(RMX_EINVAL, "bf16 element strides must be non-negative multiples of 8 (got %lld)",
                  (long long)s);
  const int64_t f4[] = {L->a_sb, L->a_ss, L->a_sh, L->ka_sb, L->ka_ss, L->ka_sh};
  for (int64_t s : f4)
    if (s < 0 || s % 4)
      return fail(RMX_EINVAL, "fp32 element strides must be non-negative multiples of 4 (got %lld)",
                  (long long)s);
  if (L->l_sb < 0 || L->l_sh < 0) return fail(RMX_EINVAL, "lse strides must be non-negative");
  return RMX_OK;
}

int check_bf16(const void* p, const char* name) {
  if (!p) return fail(RMX_EINVAL, "%s is NULL", name);
  if (!aligned(p, 16)) return fail(RMX_EINVAL, "%s must be 16-byte aligned", name);
  return RMX_OK;
}

// The attention kernels address one (batch, head) slice of a tensor with 32-bit
// byte offsets (buffer loads), up to one tile past the last row.
int check_span(int64_t rows, int64_t stride_elems, const char* name) {
  const int64_t bytes = (rows + 512) * stride_elems * 2;
  if (bytes >= ((int64_t)1 << 31))
    return fail(RMX_EINVAL, "%s: a (batch, head) slice spans %lld bytes (limit 2 GiB)", name,
                (long long)bytes);
  return RMX_OK;
}

int check_window(const rmx_attn_layout* L, int has_window, int window_right, int i) {
  if (has_window != 0 && has_window != 1)
    return fail(RMX_EINVAL, "problem %d: has_window must be 0 or 1 (got %d)", i, has_window);
  if (window_right < 0 || window_right > (1 << 28))
    return fail(RMX_EINVAL, "problem %d: window_right must lie in [0, 2^28] (got %d)", i,
                window_right);
  if (window_right != 0 && L->mask != RMX_MASK_CAUSAL)
    return fail(RMX_EINVAL, "problem %d: window_right needs RMX_MASK_CAUSAL", i);
  return RMX_OK;
}

int check_doc(const rmx_attn_layout* L, const int32_t* qg, const int32_t* kg, const int32_t* qd,
              const int32_t* kd) {
  if (L->mask != RMX_MASK_DOC) return RMX_OK;
  if (!qg || !kg || !qd || !kd)
    return fail(RMX_EINVAL, "RMX_MASK_DOC needs q_gidx, k_gidx, q_doc and k_doc");
  if (!aligned(qg, 4) || !aligned(kg, 4) || !aligned(qd, 4) || !aligned(kd, 4))
    return fail(RMX_EINVAL, "RMX_MASK_DOC index arrays must be 4-byte aligned");
  return RMX_OK;
}

}  // namespace

extern "C" {

int32_t rmx_abi_version(void) { return RMX_ABI_VERSION; }

const char* rmx_last_error(void) { return g_err.c_str(); }

int32_t rmx_attn_fwd(const rmx_attn_layout* layout, const rmx_fwd_problem* problems,
                     int32_t nproblems, void* stream) {
  int rc = check_layout(layout);
  if (rc) return rc;
  if (nproblems < 0 || (nproblems > 0 && !problems))
    return fail(RMX_EINVAL, "bad problem list (n=%d)", nproblems);
  for (int i = 0; i < nproblems; ++i) {
    const rmx_fwd_problem& p = problems[i];
    if (p.sq < 0 || p.sk < 0) return fail(RMX_EINVAL, "problem %d: negative length", i);
    if ((rc = check_window(layout, p.has_window, p.window_right, i))) return rc;
    if (p.sq == 0) continue;
    if ((rc = check_bf16(p.q, "q"))) return rc;
    if ((rc = check_span(p.sq, layout->q_ss, "q"))) return rc;
    if (p.sk > 0) {
      if ((rc = check_bf16(p.k, "k"))) return rc;
      if ((rc = check_bf16(p.v, "v"))) return rc;
      if ((rc = check_span(p.sk, layout->k_ss, "k"))) return rc;
      if ((rc = check_span(p.sk, layout->v_ss, "v"))) return rc;
    }
    if ((rc = check_doc(layout, p.q_gidx, p.k_gidx, p.q_doc, p.k_doc))) return rc;
    switch (p.mode) {
      case RMX_FWD_WRITE:
      case RMX_FWD_ACC_FINAL:
        if ((rc = check_bf16(p.out, "out"))) return rc;
        if (p.mode == RMX_FWD_ACC_FINAL && (!p.acc_out || !p.acc_lse))
          return fail(RMX_EINVAL, "problem %d: ACC_FINAL needs acc_out and acc_lse", i);
        break;
      case RMX_FWD_ACC_INIT:
      case RMX_FWD_ACC_MERGE:
        if (!p.acc_out || !p.acc_lse)
          return fail(RMX_EINVAL, "problem %d: accumulating modes need acc_out and acc_lse", i);
        break;
      default:
        return fail(RMX_EINVAL, "problem %d: unknown forward mode %d", i, p.mode);
    }
    if (p.acc_out && !aligned(p.acc_out, 16))
      return fail(RMX_EINVAL, "acc_out must be 16-byte aligned");
  }
  for (int i = 0; i < nproblems; i += RMX_MAX_BATCHED) {
    const int n = nproblems - i < RMX_MAX_BATCHED ? nproblems - i : RMX_MAX_BATCHED;
    rc = dev_status(rmx::launch_attn_fwd(*layout, problems + i, n, (hipStream_t)stream),
                    "rmx_attn_fwd launch");
    if (rc) return rc;
  }
  return RMX_OK;
}

int32_t rmx_attn_bwd_delta(const rmx_attn_layout* layout, const void* out, int32_t out_is_f32,
                           const uint16_t* dout, float* delta, const float* lse, float* nlse,
                           int32_t sq, void* stream) {
  int rc = check_layout(layout);
  if (rc) return rc;
  if (sq < 0) return fail(RMX_EINVAL, "negative sequence length");
  if (sq == 0 || layout->batch == 0) return RMX_OK;
  if ((rc = check_bf16(out, "out"))) return rc;
  if ((rc = check_bf16(dout, "dout"))) return rc;
  if (!delta) return fail(RMX_EINVAL, "delta is NULL");
  if (nlse && !lse) return fail(RMX_EINVAL, "nlse requires lse");
  return dev_status(rmx::launch_attn_bwd_delta(*layout, out, out_is_f32 != 0, dout, delta, lse,
                                               nlse, sq, (hipStream_t)stream),
                    "rmx_attn_bwd_delta launch");
}

int32_t rmx_attn_bwd(const rmx_attn_layout* layout, const rmx_bwd_problem* problems,
                     int32_t nproblems, void* stream) {
  int rc = check_layout(layout);
  if (rc) return rc;
  if (nproblems < 0 || (nproblems > 0 && !problems))
    return fail(RMX_EINVAL, "bad problem list (n=%d)", nproblems);
  for (int i = 0; i < nproblems; ++i) {
    const rmx_bwd_problem& p = problems[i];
    if (p.sq < 0 || p.sk < 0) return fail(RMX_EINVAL, "problem %d: negative length", i);
    if ((rc = check_window(layout, p.has_window, p.window_right, i))) return rc;
    if (p.sq == 0 || p.sk == 0) continue;
    if ((rc = check_bf16(p.q, "q"))) return rc;
    if ((rc = check_bf16(p.k, "k"))) return rc;
    if ((rc = check_bf16(p.v, "v"))) return rc;
    if ((rc = check_bf16(p.dout, "dout"))) return rc;
    if ((rc = check_span(p.sq, layout->q_ss, "q"))) return rc;
    if ((rc = check_span(p.sq, layout->o_ss, "dout"))) return rc;
    if ((rc = check_span(p.sk, layout->k_ss, "k"))) return rc;
    if ((rc = check_span(p.sk, layout->v_ss, "v"))) return rc;
    if (!p.lse || !p.delta) return fail(RMX_EINVAL, "problem %d: lse and delta are required", i);
    if (p.dkv_mode != RMX_GRAD_NONE && !p.nlse)
      return fail(RMX_EINVAL, "problem %d: nlse (from rmx_attn_bwd_delta) is required for dk/dv", i);
    if ((rc = check_doc(layout, p.q_gidx, p.k_gidx, p.q_doc, p.k_doc))) return rc;
    const int modes[2] = {p.dq_mode, p.dkv_mode};
    for (int m = 0; m < 2; ++m) {
      const int mode = modes[m];
      if (mode < RMX_GRAD_WRITE_BF16 || mode > RMX_GRAD_NONE)
        return fail(RMX_EINVAL, "problem %d: unknown gradient mode %d", i, mode);
      if (mode == RMX_GRAD_NONE) continue;
      const bool need_acc = mode != RMX_GRAD_WRITE_BF16;
      const bool need_bf = mode == RMX_GRAD_WRITE_BF16 || mode == RMX_GRAD_ACC_FINAL;
      if (m == 0) {
        if (need_acc && (!p.dq_acc || !aligned(p.dq_acc, 16)))
          return fail(RMX_EINVAL, "problem %d: dq_acc missing or misaligned", i);
        if (need_bf && (rc = check_bf16(p.dq, "dq"))) return rc;
      } else {
        if (need_acc && (!p.dk_acc || !p.dv_acc))
          return fail(RMX_EINVAL, "problem %d: dk_acc/dv_acc missing", i);
        if (need_bf && (!p.dk || !p.dv)) return fail(RMX_EINVAL, "problem %d: dk/dv missing", i);
      }
    }
  }
  for (int i = 0; i < nproblems; i += RMX_MAX_BATCHED) {
    const int n = nproblems - i < RMX_MAX_BATCHED ? nproblems - i : RMX_MAX_BATCHED;
    rc = dev_status(rmx::launch_attn_bwd(*layout, problems + i, n, (hipStream_t)stream),
                    "rmx_attn_bwd launch");
    if (rc) return rc;
  }
  return RMX_OK;
}

int32_t rmx_lse_merge(float* out, float* lse, const void* blk_out, int32_t blk_type,
                      const float* blk_lse, int32_t batch, int32_t seq, int32_t heads,
                      int32_t head_dim, const int64_t* o_strides, const int64_t* l_strides,
                      const int64_t* bo_strides, const int64_t* bl_strides, int32_t init,
                      void* stream) {
  if (batch < 0 || seq < 0 || heads < 0) return fail(RMX_EINVAL, "negative shape");
  if (head_dim <= 0 || head_dim % 8)
    return fail(RMX_EUNSUPPORTED, "head_dim must be a positive multiple of 8 (got %d)", head_dim);
  if (blk_type < RMX_BLK_BF16 || blk_type > RMX_BLK_F16)
    return fail(RMX_EINVAL, "unknown block type %d", blk_type);
  if ((int64_t)batch * seq * heads == 0) return RMX_OK;
  if (!out || !lse || !blk_out || !blk_lse) return fail(RMX_EINVAL, "NULL tensor pointer");
  if (!o_strides || !l_strides || !bo_strides || !bl_strides)
    return fail(RMX_EINVAL, "NULL stride array");
  if (!aligned(out, 16) || !aligned(blk_out, 16))
    return fail(RMX_EINVAL, "out and blk_out must be 16-byte aligned");
  for (int i = 0; i < 3; ++i) {
    if (o_strides[i] % 4) return fail(RMX_EINVAL, "out strides must be multiples of 4");
    if (bo_strides[i] % (blk_type == RMX_BLK_F32 ? 4 : 8))
      return fail(RMX_EINVAL, "blk_out strides must keep 16-byte alignment");
  }
  return dev_status(rmx::launch_lse_merge(out, lse, blk_out, blk_type, blk_lse, batch, seq, heads,
                                          head_dim, o_strides, l_strides, bo_strides, bl_strides,
                                          init, (hipStream_t)stream),
                    "rmx_lse_merge launch");
}

int32_t rmx_zigzag_gather(const void* src, void* dst, int32_t batch, int32_t seq, int32_t world,
                          int32_t rank, int64_t row_bytes, int64_t src_bstride,
                          const void* pad_row, void* stream) {
  if (world <= 0) return fail(RMX_EINVAL, "world must be positive (got %d)", world);
  if (rank >= world) return fail(RMX_EINVAL, "rank %d out of range for world %d", rank, world);
  if (batch < 0 || seq < 0 || row_bytes < 0) return fail(RMX_EINVAL, "negative shape");
  if ((int64_t)batch * seq == 0 || row_bytes == 0) return RMX_OK;
  if (!src || !dst) return fail(RMX_EINVAL, "NULL tensor pointer");
  if (src_bstride < (int64_t)seq * row_bytes && batch > 1)
    return fail(RMX_EINVAL, "batch stride smaller than one sequence");
  return dev_status(rmx::launch_zigzag(src, dst, batch, seq, world, rank, row_bytes, src_bstride,
                                       pad_row, 0, (hipStream_t)stream),
                    "rmx_zigzag_gather launch");
}

int32_t rmx_zigzag_scatter(const void* src, void* dst, int32_t batch, int32_t seq, int32_t world,
                           int64_t row_bytes, int64_t dst_bstride, void* stream) {
  if (world <= 0) return fail(RMX_EINVAL, "world must be positive (got %d)", world);
  if (batch < 0 || seq < 0 || row_bytes < 0) return fail(RMX_EINVAL, "negative shape");
  if ((int64_t)batch * seq == 0 || row_bytes == 0) return RMX_OK;
  if (!src || !dst) return fail(RMX_EINVAL, "NULL tensor pointer");
  if (dst_bstride < (int64_t)seq * row_bytes && batch > 1)
    return fail(RMX_EINVAL, "batch stride smaller than one sequence");
  return dev_status(rmx::launch_zigzag(src, dst, batch, seq, world, -1, row_bytes, dst_bstride,
                                       nullptr, 1, (hipStream_t)stream),
                    "rmx_zigzag_scatter launch");
}

static int check_scan(int batch, int L, int d, int groups, int world) {
  if (batch < 0 || L < 0 || d < 0) return fail(RMX_EINVAL, "negative shape");
  if (world <= 0) return fail(RMX_EINVAL, "world must be positive (got %d)", world);
  if (L % world) return fail(RMX_EINVAL, "sequence length %d not divisible by world %d", L, world);
  if (groups <= 0 || (d > 0 && d % groups))
    return fail(RMX_EINVAL, "groups (%d) must divide d (%d)", groups, d);
  return RMX_OK;
}

// The L-parallel path's plan for a validated shape; fails when the caller's workspace is
// too small or the shape does not fit its 32-bit chunk tickets.
static int scan_chunk_plan_for(rmx::ScanChunkPlan& p, int batch, int L, int d, int groups,
                               size_t workspace_bytes) {
  p = rmx::scan_chunk_plan(batch, L, d, groups);
  if ((int64_t)batch * p.ntiles * p.nchunks >= ((int64_t)1 << 31))
    return fail(RMX_EINVAL, "%lld chunks exceed the chained scan's 2^31 tickets",
                (long long)batch * p.ntiles * p.nchunks);
  if (workspace_bytes < p.bytes)
    return fail(RMX_EINVAL, "workspace of %zu bytes is below the %zu the L-parallel scan needs",
                workspace_bytes, p.bytes);
  return RMX_OK;
}

size_t rmx_linear_scan_workspace(int32_t batch, int32_t L, int32_t d, int32_t groups,
                                 int32_t* chunk_tokens) {
  if (batch <= 0 || L <= 0 || d <= 0 || groups <= 0 || d % groups) {
    if (chunk_tokens) *chunk_tokens = 0;
    return 0;
  }
  const rmx::ScanChunkPlan p = rmx::scan_chunk_plan(batch, L, d, groups);
  if (chunk_tokens) *chunk_tokens = p.TC;
  return p.bytes;
}

int32_t rmx_linear_scan_status(const void* workspace, size_t workspace_bytes, void* stream) {
  if (!workspace) return RMX_OK;
  if (workspace_bytes < 256) return fail(RMX_EINVAL, "workspace of %zu bytes is too small", workspace_bytes);
  hipError_t e;
  const int flag = rmx::read_linear_scan_failure(workspace, (hipStream_t)stream, &e);
  if (e != hipSuccess) return dev_status(e, "linear scan status");
  if (flag)
    return fail(RMX_EDEVICE, "the L-parallel linear scan's look-back gave up waiting for a chunk "
                             "(its outputs hold NaN)");
  return RMX_OK;
}

int32_t rmx_linear_scan_fwd(const float* a, const float* b, const float* h_in, float* h,
                            float* chunk_state, int32_t batch, int32_t L, int32_t d, int32_t groups,
                            int32_t world, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_scan(batch, L, d, groups, world);
  if (rc) return rc;
  if ((int64_t)batch * L * d == 0) return RMX_OK;
  if (!a || !b || !h) return fail(RMX_EINVAL, "NULL tensor pointer");
  if (!aligned(a, 16) || !aligned(b, 16) || !aligned(h, 16) || (h_in && !aligned(h_in, 16)))
    return fail(RMX_EINVAL, "a, b, h_in and h must be 16-byte aligned");
  if (workspace) {
    rmx::ScanChunkPlan p;
    if ((rc = scan_chunk_plan_for(p, batch, L, d, groups, workspace_bytes))) return rc;
    if (chunk_state && (L / world) % p.TC)
      return fail(RMX_EINVAL,
                  "chunk_state with the L-parallel scan needs L / world (%d) to be a multiple "
                  "of its %d-token chunks (run it without a workspace)", L / world, p.TC);
    return dev_status(rmx::launch_linear_scan_fwd_chunked(p, a, b, h_in, h, chunk_state, workspace,
                                                          batch, L, d, groups, world,
                                                          (hipStream_t)stream),
                      "rmx_linear_scan_fwd launch");
  }
  return dev_status(
      rmx::launch_linear_scan_fwd(a, b, h_in, h, chunk_state, batch, L, d, groups, world,
                                  (hipStream_t)stream),
      "rmx_linear_scan_fwd launch");
}

int32_t rmx_linear_scan_bwd(const float* a, const float* h, const float* h_in, const float* dh,
                            float* da, float* db, float* dh_in, int32_t batch, int32_t L,
                            int32_t d, int32_t groups, int32_t world, void* workspace,
                            size_t workspace_bytes, void* stream) {
  int rc = check_scan(batch, L, d, groups, world);
  if (rc) return rc;
  if ((int64_t)batch * d == 0) return RMX_OK;
  if (L == 0) {
    if (dh_in && !aligned(dh_in, 16)) return fail(RMX_EINVAL, "dh_in must be 16-byte aligned");
    return dev_status(rmx::launch_linear_scan_bwd(a, h, h_in, dh, da, db, dh_in, batch, L, d,
                                                  groups, world, (hipStream_t)stream),
                      "rmx_linear_scan_bwd launch");
  }
  if (!a || !h || !dh || !da || !db) return fail(RMX_EINVAL, "NULL tensor pointer");
  if (!aligned(a, 16) || !aligned(h, 16) || !aligned(dh, 16) || !aligned(da, 16) ||
      !aligned(db, 16) || (h_in && !aligned(h_in, 16)) || (dh_in && !aligned(dh_in, 16)))
    return fail(RMX_EINVAL, "scan tensors must be 16-byte aligned");
  if (dh_in && !h_in)
    return fail(RMX_EINVAL, "dh_in is the gradient of h_in: pass the forward's h_in with it");
  if (workspace) {
    rmx::ScanChunkPlan p;
    if ((rc = scan_chunk_plan_for(p, batch, L, d, groups, workspace_bytes))) return rc;
    return dev_status(rmx::launch_linear_scan_bwd_chunked(p, a, h, h_in, dh, da, db, dh_in,
                                                          workspace, batch, L, d, groups,
                                                          (hipStream_t)stream),
                      "rmx_linear_scan_bwd launch");
  }
  return dev_status(rmx::launch_linear_scan_bwd(a, h, h_in, dh, da, db, dh_in, batch, L, d,
                                                groups, world, (hipStream_t)stream),
                    "rmx_linear_scan_bwd launch");
}

int32_t rmx_mamba2_cp_correction(const uint16_t* out, uint16_t* y, const float* h_final,
                                 float* h_final_out, const uint16_t* C, const float* cum_A,
                                 const float* h_prev, const int32_t* seq_idx, int32_t batch,
                                 int32_t T, int32_t nheads, int32_t head_dim, int32_t ngroups,
                                 int32_t d_state, void* stream) {
  if (batch < 0 || T < 0 || nheads < 0) return fail(RMX_EINVAL, "negative shape");
  if (head_dim != 32 && head_dim != 64 && head_dim != 128)
    return fail(RMX_EUNSUPPORTED, "head_dim must be 32, 64 or 128 (got %d)", head_dim);
  if (d_state != 16 && d_state != 32 && d_state != 64 && d_state != 128 && d_state != 256)
    return fail(RMX_EUNSUPPORTED, "d_state must be 16, 32, 64, 128 or 256 (got %d)", d_state);
  if ((int64_t)head_dim * d_state > 32768)
    return fail(RMX_EUNSUPPORTED, "head_dim * d_state must be at most 32768 (got %d x %d)",
                head_dim, d_state);
  if (ngroups <= 0 || nheads % ngroups)
    return fail(RMX_EINVAL, "ngroups (%d) must divide nheads (%d)", ngroups, nheads);
  if ((int64_t)batch * nheads == 0) return RMX_OK;
  if (T == 0) return fail(RMX_EINVAL, "the shard has no tokens (T == 0)");
  if (!out || !y || !h_final || !h_final_out || !C || !cum_A || !h_prev)
    return fail(RMX_EINVAL, "NULL tensor pointer");
  if (!aligned(C, 16) || !aligned(h_prev, 16) || !aligned(h_final, 16) || !aligned(h_final_out, 16) ||
      !aligned(out, 16) || !aligned(y, 16))
    return fail(RMX_EINVAL, "out, y, C, h_prev, h_final and h_final_out must be 16-byte aligned");
  return dev_status(rmx::launch_mamba2_correction(out, y, h_final, h_final_out, C, cum_A, h_prev,
                                                  seq_idx, batch, T, nheads, head_dim, ngroups,
                                                  d_state, (hipStream_t)stream),
                    "rmx_mamba2_cp_correction launch");
}

static int check_mamba_bwd(int32_t batch, int32_t T, int32_t nheads, int32_t head_dim,
                           int32_t ngroups, int32_t d_state) {
  if (batch < 0 || T < 0 || nheads < 0) return fail(RMX_EINVAL, "negative shape");
  if (head_dim != 64 && head_dim != 128)
    return fail(RMX_EUNSUPPORTED, "the correction backward takes head_dim 64 or 128 (got %d)", head_dim);
  if (d_state != 64 && d_state != 128)
    return fail(RMX_EUNSUPPORTED, "the correction backward takes d_state 64 or 128 (got %d)", d_state);
  if (ngroups <= 0 || nheads % ngroups)
    return fail(RMX_EINVAL, "ngroups (%d) must divide nheads (%d)", ngroups, nheads);
  const int heads_per_wg = head_dim == 64 ? 4 : 2;
  if ((nheads / ngroups) % heads_per_wg)
    return fail(RMX_EUNSUPPORTED,
                "the correction backward needs nheads / ngroups divisible by %d at head_dim %d",
                heads_per_wg, head_dim);
  const int64_t row = std::max<int64_t>({(int64_t)nheads * head_dim * 2,
                                         (int64_t)ngroups * d_state * 2, (int64_t)nheads * 4});
  if (((int64_t)T + 256) * row >= ((int64_t)1 << 31))
    return fail(RMX_EUNSUPPORTED, "a batch row of the shard exceeds 2 GiB");
  return RMX_OK;
}

size_t rmx_mamba2_cp_correction_bwd_workspace(int32_t batch, int32_t T, int32_t nheads,
                                              int32_t head_dim, int32_t ngroups, int32_t d_state) {
  if (check_mamba_bwd(batch, T, nheads, head_dim, ngroups, d_state)) return 0;
  return rmx::mamba2_bwd_workspace(batch, T, nheads, head_dim, d_state);
}

// Shared argument checks of the two correction-backward entry points (1 = nothing to do).
static int check_mamba_bwd_args(const uint16_t* gy, const float* ghf, const uint16_t* C,
                                const float* cum_A, const float* h_prev, uint16_t* gC,
                                float* g_cumA, float* g_hprev, int32_t batch, int32_t T,
                                int32_t nheads, int32_t head_dim, int32_t ngroups,
                                int32_t d_state) {
  int rc = check_mamba_bwd(batch, T, nheads, head_dim, ngroups, d_state);
  if (rc) return rc;
  if ((int64_t)batch * nheads == 0) return 1;
  if (T == 0) return fail(RMX_EINVAL, "the shard has no tokens (T == 0)");
  if (!gy || !C || !cum_A || !h_prev || !gC || !g_cumA || !g_hprev)
    return fail(RMX_EINVAL, "NULL tensor pointer");
  if (!aligned(gy, 16) || !aligned(C, 16) || !aligned(h_prev, 16) || !aligned(gC, 16) ||
      !aligned(g_hprev, 16) || (ghf && !aligned(ghf, 16)))
    return fail(RMX_EINVAL, "gy, C, h_prev, ghf, gC and g_hprev must be 16-byte aligned");
  return RMX_OK;
}

int32_t rmx_mamba2_cp_correction_bwd(const uint16_t* gy, const float* ghf, const uint16_t* C,
                                     const float* cum_A, const float* h_prev,
                                     const int32_t* seq_idx, uint16_t* gC, float* g_cumA,
                                     float* g_hprev, void* workspace, size_t workspace_bytes,
                                     int32_t batch, int32_t T, int32_t nheads, int32_t head_dim,
                                     int32_t ngroups, int32_t d_state, void* stream) {
  int rc = check_mamba_bwd_args(gy, ghf, C, cum_A, h_prev, gC, g_cumA, g_hprev, batch, T, nheads,
                                head_dim, ngroups, d_state);
  if (rc) return rc < 0 ? rc : RMX_OK;
  if (!workspace) return fail(RMX_EINVAL, "NULL workspace");
  const size_t need = rmx::mamba2_bwd_workspace(batch, T, nheads, head_dim, d_state);
  if (workspace_bytes < need)
    return fail(RMX_EINVAL, "workspace of %zu bytes is below the %zu required", workspace_bytes, need);
  return dev_status(rmx::launch_mamba2_correction_bwd(gy, ghf, C, cum_A, h_prev, seq_idx, gC, g_cumA,
                                                      g_hprev, workspace, batch, T, nheads,
                                                      head_dim, ngroups, d_state,
                                                      (hipStream_t)stream),
                    "rmx_mamba2_cp_correction_bwd launch");
}

int32_t rmx_mamba2_cp_correction_bwd_noalloc(const uint16_t* gy, const float* ghf,
                                             const uint16_t* C, const float* cum_A,
                                             const float* h_prev, const int32_t* seq_idx,
                                             uint16_t* gC, float* g_cumA, float* g_hprev,
                                             int32_t batch, int32_t T, int32_t nheads,
                                             int32_t head_dim, int32_t ngroups, int32_t d_state,
                                             void* stream) {
  int rc = check_mamba_bwd_args(gy, ghf, C, cum_A, h_prev, gC, g_cumA, g_hprev, batch, T, nheads,
                                head_dim, ngroups, d_state);
  if (rc) return rc < 0 ? rc : RMX_OK;
  const size_t need = rmx::mamba2_bwd_workspace(batch, T, nheads, head_dim, d_state);
  if (need > RMX_MAMBA2_BWD_SCRATCH_MAX)
    return fail(RMX_EINVAL,
                "the shape needs a %zu-byte workspace, above the %zu bytes of the allocation-free "
                "entry point's scratch array (use rmx_mamba2_cp_correction_bwd with a workspace)",
                need, (size_t)RMX_MAMBA2_BWD_SCRATCH_MAX);
  // the scratch array is per device: the stream must run on the current one
  int cur = 0;
  if ((rc = dev_status(hipGetDevice(&cur), "hipGetDevice"))) return rc;
  if (stream) {
    hipDevice_t sd = 0;
    if ((rc = dev_status(hipStreamGetDevice((hipStream_t)stream, &sd), "hipStreamGetDevice")))
      return rc;
    if ((int)sd != cur)
      return fail(RMX_EINVAL,
                  "the stream belongs to device %d but the current device is %d (the "
                  "allocation-free entry point uses the current device's scratch array)",
                  (int)sd, cur);
  }
  void* ws = nullptr;
  rc = dev_status(rmx::mamba2_bwd_scratch(&ws), "scratch array lookup (hipGetSymbolAddress)");
  if (rc) return rc;
  return dev_status(rmx::launch_mamba2_correction_bwd(gy, ghf, C, cum_A, h_prev, seq_idx, gC, g_cumA,
                                                      g_hprev, ws, batch, T, nheads, head_dim,
                                                      ngroups, d_state, (hipStream_t)stream),
                    "rmx_mamba2_cp_correction_bwd_noalloc launch");
}

static int check_dt(const void* dt, int32_t dt_is_f32, const float* A, int32_t softplus,
                    int32_t rows, int32_t T, int32_t nheads) {
  if (rows < 0 || T < 0 || nheads < 0) return fail(RMX_EINVAL, "negative rows, T or nheads");
  if (dt_is_f32 != 0 && dt_is_f32 != 1) return fail(RMX_EINVAL, "dt_is_f32 must be 0 or 1");
  if (softplus != 0 && softplus != 1) return fail(RMX_EINVAL, "dt_softplus must be 0 or 1");
  if ((int64_t)rows * T * nheads == 0) return RMX_OK;
  if (!dt || !A) return fail(RMX_EINVAL, "NULL tensor pointer");
  if ((int64_t)rows * ((nheads + 63) / 64) > 2147483647LL)
    return fail(RMX_EUNSUPPORTED, "more than 2^31 workgroups");
  return RMX_OK;
}

int32_t rmx_mamba2_dt_cumsum(const void* dt, int32_t dt_is_f32, const float* dt_bias,
                             const float* A, int32_t dt_softplus, float* cum_A, float* e,
                             float* decay, int32_t rows, int32_t T, int32_t nheads, void* stream) {
  int rc = check_dt(dt, dt_is_f32, A, dt_softplus, rows, T, nheads);
  if (rc) return rc;
  if ((int64_t)rows * T * nheads == 0) return RMX_OK;
  if (!cum_A || !decay) return fail(RMX_EINVAL, "NULL tensor pointer");
  return dev_status(rmx::launch_mamba2_dt_cumsum(dt, dt_is_f32, dt_bias, A, dt_softplus, cum_A,
                                                 e, decay, rows, T, nheads, (hipStream_t)stream),
                    "rmx_mamba2_dt_cumsum launch");
}

int32_t rmx_mamba2_dt_cumsum_bwd(const void* dt, int32_t dt_is_f32, const float* dt_bias,
                                 const float* A, int32_t dt_softplus, const float* g_cum_A,
                                 const float* g_e, const float* g_decay, const float* decay,
                                 float* g_dt, float* g_A, float* g_dt_bias, int32_t rows,
                                 int32_t T, int32_t nheads, void* stream) {
  int rc = check_dt(dt, dt_is_f32, A, dt_softplus, rows, T, nheads);
  if (rc) return rc;
  if ((int64_t)rows * T * nheads == 0) return RMX_OK;
  if (!g_dt || !g_A || (g_decay && !decay)) return fail(RMX_EINVAL, "NULL tensor pointer");
  return dev_status(rmx::launch_mamba2_dt_cumsum_bwd(dt, dt_is_f32, dt_bias, A, dt_softplus,
                                                     g_cum_A, g_e, g_decay, decay, g_dt, g_A,
                                                     g_dt_bias, rows, T, nheads,
                                                     (hipStream_t)stream),
                    "rmx_mamba2_dt_cumsum_bwd launch");
}

static int check_state(const uint16_t* x, const uint16_t* B, const float* e, const float* cum_A,
                       int32_t rows, int32_t T, int32_t H, int32_t D, int32_t G, int32_t N) {
  if (rows < 0 || T < 0 || H < 0 || G < 1) return fail(RMX_EINVAL, "bad rows, T, nheads or ngroups");
  if ((D != 64 && D != 128) || (N != 64 && N != 128))
    return fail(RMX_EUNSUPPORTED, "head_dim %d / d_state %d outside {64, 128}", D, N);
  if (H % G) return fail(RMX_EINVAL, "nheads %d not a multiple of ngroups %d", H, G);
  if ((int64_t)rows * T * H == 0) return RMX_OK;
  // 32-bit byte offsets per row, with a tile of slack past the end
  if ((int64_t)(T + 256) * H * D * 2 >= 2147483647LL || (int64_t)(T + 256) * G * N * 2 >= 2147483647LL)
    return fail(RMX_EUNSUPPORTED, "more than 2^31 bytes of x or B per row");
  if ((int64_t)rows * H * 2 > 2147483647LL || (int64_t)rows * G * ((T + 255) / 256) > 2147483647LL)
    return fail(RMX_EUNSUPPORTED, "more than 2^31 workgroups");
  if (!x || !B || !e || !cum_A) return fail(RMX_EINVAL, "NULL tensor pointer");
  if (!aligned(x, 16) || !aligned(B, 16)) return fail(RMX_EINVAL, "x and B must be 16-byte aligned");
  return RMX_OK;
}

int32_t rmx_mamba2_chunk_state(const uint16_t* x, const uint16_t* B, const float* e,
                               const float* cum_A, const int32_t* t0, float* state, int32_t rows,
                               int32_t T, int32_t nheads, int32_t head_dim, int32_t ngroups,
                               int32_t d_state, void* stream) {
  int rc = check_state(x, B, e, cum_A, rows, T, nheads, head_dim, ngroups, d_state);
  if (rc) return rc;
  if ((int64_t)rows * nheads == 0) return RMX_OK;
  if (!state) return fail(RMX_EINVAL, "NULL tensor pointer");
  return dev_status(rmx::launch_mamba2_chunk_state(x, B, e, cum_A, t0, state, rows, T, nheads,
                                                   head_dim, ngroups, d_state,
                                                   (hipStream_t)stream),
                    "rmx_mamba2_chunk_state launch");
}

size_t rmx_mamba2_chunk_state_bwd_workspace(int32_t rows, int32_t nheads, int32_t head_dim,
                                            int32_t d_state) {
  if (rows <= 0 || nheads <= 0) return 0;
  if ((head_dim != 64 && head_dim != 128) || (d_state != 64 && d_state != 128)) return 0;
  return rmx::mamba2_chunk_state_bwd_workspace(rows, nheads, head_dim, d_state);
}

int32_t rmx_mamba2_chunk_state_bwd(const uint16_t* x, const uint16_t* B, const float* e,
                                   const float* cum_A, const int32_t* t0, const float* g_state,
                                   uint16_t* g_x, uint16_t* g_B, float* g_e, float* g_cum_A,
                                   int32_t rows, int32_t T, int32_t nheads, int32_t head_dim,
                                   int32_t ngroups, int32_t d_state, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  int rc = check_state(x, B, e, cum_A, rows, T, nheads, head_dim, ngroups, d_state);
  if (rc) return rc;
  if ((int64_t)rows * T * nheads == 0) return RMX_OK;
  if (!g_state || !g_x || !g_B || !g_e || !g_cum_A) return fail(RMX_EINVAL, "NULL tensor pointer");
  if (!aligned(g_state, 16) || !aligned(g_x, 8) || !aligned(g_B, 8))
    return fail(RMX_EINVAL, "g_state must be 16-byte and g_x, g_B 8-byte aligned");
  const size_t need = rmx::mamba2_chunk_state_bwd_workspace(rows, nheads, head_dim, d_state);
  if (workspace && need > 0) {
    if (workspace_bytes < need)
      return fail(RMX_EINVAL, "workspace of %zu bytes, %zu needed", workspace_bytes, need);
    if (!aligned(workspace, 16)) return fail(RMX_EINVAL, "workspace must be 16-byte aligned");
    if ((int64_t)T * nheads * head_dim * 2 >= ((int64_t)1 << 31))
      return fail(RMX_EINVAL, "a row of x spans 2 GiB or more");
  }
  return dev_status(rmx::launch_mamba2_chunk_state_bwd(x, B, e, cum_A, t0, g_state, g_x, g_B,
                                                       g_e, g_cum_A, rows, T, nheads, head_dim,
                                                       ngroups, d_state, need > 0 ? workspace : nullptr,
                                                       (hipStream_t)stream),
                    "rmx_mamba2_chunk_state_bwd launch");
}

static int check_conv(const uint16_t* x, const uint16_t* weight, const uint16_t* bias,
                      const void* y, int32_t world, int32_t batch, int32_t channels,
                      int32_t local_len, int32_t width, int32_t activation) {
  if (world < 1) return fail(RMX_EINVAL, "world must be positive (got %d)", world);
  if (batch < 0 || channels < 0 || local_len < 0)
    return fail(RMX_EINVAL, "negative batch, channels or length");
  if (width < 1 || width > 9)
    return fail(RMX_EUNSUPPORTED, "convolution width %d outside 1..9", width);
  if (local_len % 8)
    return fail(RMX_EUNSUPPORTED, "local length %d is not a multiple of 8", local_len);
  if (activation != 0 && activation != 1)
    return fail(RMX_EINVAL, "unknown activation %d (0 none, 1 silu)", activation);
  if ((int64_t)batch * channels * local_len == 0) return RMX_OK;
  if ((int64_t)world * batch * channels * ((local_len / 8 + 255) / 256) > 2147483647LL)
    return fail(RMX_EUNSUPPORTED, "conv grid of more than 2^31 workgroups");
  if (!x || !weight || !y) return fail(RMX_EINVAL, "NULL tensor pointer");
  if (!aligned(x, 16) || !aligned(y, 16)) return fail(RMX_EINVAL, "x and outputs must be 16-byte aligned");
  if (!aligned(weight, 2) || (bias && !aligned(bias, 2)))
    return fail(RMX_EINVAL, "weight and bias must be 2-byte aligned");
  return RMX_OK;
}

int32_t rmx_causal_conv1d_cp(const uint16_t* x, const uint16_t* weight, const uint16_t* bias,
                             const int32_t* doc, uint16_t* y, int32_t world, int32_t batch,
                             int32_t channels, int32_t local_len, int32_t width,
                             int32_t activation, void* stream) {
  int rc = check_conv(x, weight, bias, y, world, batch, channels, local_len, width, activation);
  if (rc) return rc;
  if ((int64_t)batch * channels * local_len == 0) return RMX_OK;
  return dev_status(rmx::launch_causal_conv1d_cp(x, weight, bias, doc, y, world, batch, channels,
                                                 local_len, width, activation, (hipStream_t)stream),
                    "rmx_causal_conv1d_cp launch");
}

int32_t rmx_causal_conv1d_cp_bwd(const uint16_t* x, const uint16_t* weight, const uint16_t* bias,
                                 const int32_t* doc, const uint16_t* dy, uint16_t* dx,
                                 float* dweight, float* dbias, int32_t world, int32_t batch,
                                 int32_t channels, int32_t local_len, int32_t width,
                                 int32_t activation, void* stream) {
  int rc = check_conv(x, weight, bias, dx, world, batch, channels, local_len, width, activation);
  if (rc) return rc;
  if ((int64_t)batch * channels * local_len == 0) return RMX_OK;
  if (!dy || !dweight) return fail(RMX_EINVAL, "NULL tensor pointer");
  if (!aligned(dy, 16)) return fail(RMX_EINVAL, "dy must be 16-byte aligned");
  return dev_status(rmx::launch_causal_conv1d_cp_bwd(x, weight, bias, doc, dy, dx, dweight, dbias,
                                                     world, batch, channels, local_len, width,
                                                     activation, (hipStream_t)stream),
                    "rmx_causal_conv1d_cp_bwd launch");
}

}  // extern "C"
