// C-ABI entry points of libqhtp: argument validation, error reporting and dispatch to the
// kernel launchers.  Modelled on the reference's prepared-run ABI
// (example/handwritten_hmx_matmul/include/handwritten_hmx_matmul.h:11-52), with the
// difference that an unsupported or invalid shape is always reported, never silently skipped
// (the reference's QHPI callbacks return success without writing, e.g.
// HmxU8I8ToU8MatMulOp.cpp:230,246,500,550).

#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "qmm_internal.h"

namespace {
thread_local char g_err[512] = "";
}

namespace qh {

qh_status fail(qh_status st, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return st;
}

qh_status hip_fail(hipError_t err, const char *what) {
  return fail(QH_STATUS_RUNTIME_ERROR, "%s: %s", what, hipGetErrorString(err));
}

}  // namespace qh

using namespace qh;

extern "C" {

const char *qh_status_string(qh_status status) {
  switch (status) {
    case QH_STATUS_OK:
      return "ok";
    case QH_STATUS_INVALID_ARGUMENT:
      return "invalid_argument";
    case QH_STATUS_UNSUPPORTED:
      return "unsupported";
    case QH_STATUS_RUNTIME_ERROR:
      return "runtime_error";
    case QH_STATUS_SHAPE_UNSUPPORTED:
      return "shape_unsupported";
  }
  return "unknown";
}

const char *qh_last_error(void) { return g_err; }

uint32_t qh_version(void) { return 0x000100u; }

qh_status qh_qmm_run_path(const qh_qmm_prepared *prep, uint32_t m, const void *act_dev, void *out_dev,
                          uint32_t path, void *stream) {
  if (prep == nullptr) return fail(QH_STATUS_INVALID_ARGUMENT, "qh_qmm_run: prepared handle is NULL");
  if (m == 0) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_qmm_run: M must be >= 1");
  if (m > (1u << 24)) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_qmm_run: M=%u too large", m);
  if (act_dev == nullptr || out_dev == nullptr) return fail(QH_STATUS_INVALID_ARGUMENT, "qh_qmm_run: NULL buffer");
  const size_t ea = prep->shape.act_bits == 16 ? 2 : 1;
  if (reinterpret_cast<uintptr_t>(act_dev) % 16 || (static_cast<size_t>(prep->shape.K) * ea) % 16)
    return fail(QH_STATUS_INVALID_ARGUMENT, "qh_qmm_run: activation rows must be 16-byte aligned");
  if (path > 2) return fail(QH_STATUS_INVALID_ARGUMENT, "qh_qmm_run: unknown path %u", path);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (prep->shape.exact_only) {
    if (prep->shape.wfmt == QH_WEIGHT_I16)
      return fail(QH_STATUS_UNSUPPORTED, "qh_qmm_run: int16 weights have no float requantisation; use qh_qmm_run_contract");
    // per-group weights: the exact integer GEMM for every M (path ignored)
    return launch_qmm_exact(prep, static_cast<int>(m), act_dev, out_dev, 0, 0, 1, s);
  }
  const bool gemv = path == 2 || (path == 0 && m <= 16 && gemv_fits(prep, static_cast<int>(m)));
  if (gemv) return launch_qmm_gemv(prep, static_cast<int>(m), act_dev, out_dev, s);
  return launch_qmm_gemm(prep, static_cast<int>(m), act_dev, out_dev, s);
}

qh_status qh_qmm_run(const qh_qmm_prepared *prep, uint32_t m, const void *act_dev, void *out_dev, void *stream) {
  return qh_qmm_run_path(prep, m, act_dev, out_dev, 0, stream);
}

qh_status qh_qmm_accumulate(const qh_qmm_prepared *prep, uint32_t m, const void *act_dev, int64_t *acc_dev,
                            void *stream) {
  if (prep == nullptr) return fail(QH_STATUS_INVALID_ARGUMENT, "qh_qmm_accumulate: prepared handle is NULL");
  if (m == 0 || m > (1u << 24)) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_qmm_accumulate: bad M=%u", m);
  if (act_dev == nullptr || acc_dev == nullptr)
    return fail(QH_STATUS_INVALID_ARGUMENT, "qh_qmm_accumulate: NULL buffer");
  if (reinterpret_cast<uintptr_t>(act_dev) % 16)
    return fail(QH_STATUS_INVALID_ARGUMENT, "qh_qmm_accumulate: activation must be 16-byte aligned");
  if (prep->shape.exact_only)
    return launch_qmm_exact(prep, static_cast<int>(m), act_dev, acc_dev, 1, 0, 1, static_cast<hipStream_t>(stream));
  return launch_qmm_accumulate(prep, static_cast<int>(m), act_dev, acc_dev, static_cast<hipStream_t>(stream));
}

namespace {

// Validates a contract and its divisor; *param = the value the kernels take.
qh_status contract_param(const char *fn, uint32_t contract, uint32_t divisor, uint32_t *param) {
  if (contract > QH_CONTRACT_U8_DRAIN) return fail(QH_STATUS_UNSUPPORTED, "%s: unknown contract %u", fn, contract);
  const bool divides = contract == QH_CONTRACT_DIV_RINT || contract == QH_CONTRACT_FLOOR256_DIV_RINT ||
                       contract == QH_CONTRACT_ROUND_DIV;
  if (divides && (divisor == 0 || divisor > (1u << 30)))
    return fail(QH_STATUS_INVALID_ARGUMENT, "%s: divisor %u must be in [1, 2^30]", fn, divisor);
  if (contract == QH_CONTRACT_U8_DRAIN && ((divisor >> 10) & 31u) == 31u)
    return fail(QH_STATUS_INVALID_ARGUMENT, "%s: drain scale 0x%04x is not a finite half", fn, divisor & 0xFFFFu);
  *param = divides || contract == QH_CONTRACT_U8_DRAIN ? divisor : 1u;
  return QH_STATUS_OK;
}

}  // namespace

qh_status qh_qmm_run_contract(const qh_qmm_prepared *prep, uint32_t m, const void *act_dev, void *out_dev,
                              uint32_t contract, uint32_t divisor, void *stream) {
  if (prep == nullptr) return fail(QH_STATUS_INVALID_ARGUMENT, "qh_qmm_run_contract: prepared handle is NULL");
  if (m == 0 || m > (1u << 22)) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_qmm_run_contract: bad M=%u", m);
  if (act_dev == nullptr || out_dev == nullptr)
    return fail(QH_STATUS_INVALID_ARGUMENT, "qh_qmm_run_contract: NULL buffer");
  if (reinterpret_cast<uintptr_t>(act_dev) % 16)
    return fail(QH_STATUS_INVALID_ARGUMENT, "qh_qmm_run_contract: activation must be 16-byte aligned");
  uint32_t param = 1;
  const qh_status st = contract_param("qh_qmm_run_contract", contract, divisor, &param);
  if (st != QH_STATUS_OK) return st;
  return launch_qmm_exact(prep, static_cast<int>(m), act_dev, out_dev, 2, static_cast<int>(contract),
                          static_cast<int>(param), static_cast<hipStream_t>(stream));
}

qh_status qh_qmm_run_chain(const qh_qmm_prepared *prep, uint32_t m, uint32_t chain, const void *act_dev,
                           void *out_dev, void *scratch_dev, uint32_t contract, uint32_t divisor, void *stream) {
  if (prep == nullptr) return fail(QH_STATUS_INVALID_ARGUMENT, "qh_qmm_run_chain: prepared handle is NULL");
  if (chain == 0 || chain > 4096) return fail(QH_STATUS_INVALID_ARGUMENT, "qh_qmm_run_chain: chain=%u", chain);
  if (act_dev == nullptr || out_dev == nullptr) return fail(QH_STATUS_INVALID_ARGUMENT, "qh_qmm_run_chain: NULL buffer");
  const QmmShape &sh = prep->shape;
  if (chain > 1) {
    if (sh.K != sh.N || sh.act_bits != sh.out_bits)
      return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_qmm_run_chain: chain > 1 needs K == N and act_bits == out_bits");
    if (scratch_dev == nullptr) return fail(QH_STATUS_INVALID_ARGUMENT, "qh_qmm_run_chain: chain > 1 needs scratch");
    if (reinterpret_cast<uintptr_t>(out_dev) % 16 || reinterpret_cast<uintptr_t>(scratch_dev) % 16)
      return fail(QH_STATUS_INVALID_ARGUMENT, "qh_qmm_run_chain: out and scratch must be 16-byte aligned");
    // the three byte ranges must not overlap: act [M x K], out and scratch [M x N] each
    const uintptr_t a = reinterpret_cast<uintptr_t>(act_dev), o = reinterpret_cast<uintptr_t>(out_dev),
                    s = reinterpret_cast<uintptr_t>(scratch_dev);
    const uintptr_t na = static_cast<uintptr_t>(m) * sh.K * (sh.act_bits == 16 ? 2 : 1);
    const uintptr_t no = static_cast<uintptr_t>(m) * sh.N * (sh.out_bits == 16 ? 2 : 1);
    auto overlap = [](uintptr_t p, uintptr_t np, uintptr_t q, uintptr_t nq) { return p < q + nq && q < p + np; };
    if (overlap(a, na, o, no) || overlap(a, na, s, no) || overlap(o, no, s, no))
      return fail(QH_STATUS_INVALID_ARGUMENT, "qh_qmm_run_chain: act, out and scratch ranges must not overlap");
  }
  if (chain > 1 && contract != QH_CONTRACT_NONE && chain_fusable(prep)) {
    // every step in one launch: the intermediate activations stay on chip (scratch unused)
    if (m == 0 || m > (1u << 22)) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_qmm_run_chain: bad M=%u", m);
    if (reinterpret_cast<uintptr_t>(act_dev) % 16)
      return fail(QH_STATUS_INVALID_ARGUMENT, "qh_qmm_run_chain: activation must be 16-byte aligned");
    uint32_t param = 1;
    const qh_status st = contract_param("qh_qmm_run_chain", contract, divisor, &param);
    if (st != QH_STATUS_OK) return st;
    return launch_qmm_chain(prep, static_cast<int>(m), static_cast<int>(chain), act_dev, out_dev,
                            static_cast<int>(contract), static_cast<int>(param), static_cast<hipStream_t>(stream));
  }
  const void *src = act_dev;
  for (uint32_t i = 0; i < chain; ++i) {
    // the last step writes out_dev; earlier steps alternate backwards from there
    void *dst = ((chain - 1 - i) % 2 == 0) ? out_dev : scratch_dev;
    const qh_status st = contract == QH_CONTRACT_NONE
                             ? qh_qmm_run(prep, m, src, dst, stream)
                             : qh_qmm_run_contract(prep, m, src, dst, contract, divisor, stream);
    if (st != QH_STATUS_OK) return st;
    src = dst;
  }
  return QH_STATUS_OK;
}

qh_status qh_qmm_query(const qh_qmm_prepared *prep, qh_qmm_info *info) {
  if (prep == nullptr || info == nullptr) return fail(QH_STATUS_INVALID_ARGUMENT, "qh_qmm_query: NULL argument");
  const QmmShape &sh = prep->shape;
  info->k = static_cast<uint32_t>(sh.K);
  info->n = static_cast<uint32_t>(sh.N);
  info->act_bits = static_cast<uint32_t>(sh.act_bits);
  info->out_bits = static_cast<uint32_t>(sh.out_bits);
  info->weight_format = static_cast<uint32_t>(sh.wfmt);
  info->lpbq_block = static_cast<uint32_t>(sh.lpbq_block);
  info->device_bytes = prep->device_bytes;
  info->gemm_weight_bytes = prep->gemm_weight_bytes;
  info->gemv_weight_bytes = prep->gemv_weight_bytes;
  return QH_STATUS_OK;
}

qh_status qh_qmm_release(qh_qmm_prepared *prep) {
  if (prep == nullptr) return QH_STATUS_OK;
  int cur = 0;
  (void)hipGetDevice(&cur);
  (void)hipSetDevice(prep->device_id);
  hipError_t err = hipDeviceSynchronize();
  QmmDevice &D = prep->dev;
  void *ptrs[] = {D.tiles, D.gemv_tiles, D.gemv_lpbq, D.alpha, D.beta, D.corr,
                  D.margin, D.absb, D.bias_deq, D.s32, D.mant, D.colsum, D.gemv_margin_r1,
                  D.colsum_r, D.alpha_e, D.scale_exp, D.margin_exact, D.resid, D.bias_q,
                  D.corr_int, D.mult, D.corr_rq, D.s32g, D.margin_lo, D.lpbq_nk, D.gemv_rec};
  for (void *p : ptrs)
    if (p) (void)hipFree(p);
  (void)hipSetDevice(cur);
  delete prep;
  if (err != hipSuccess) return hip_fail(err, "qh_qmm_release");
  return QH_STATUS_OK;
}

qh_status qh_w4_lpbq_expand_to_i8(const uint8_t *weight_lpbq_dev, const uint8_t *block_scale_dev,
                                  uint8_t *expanded_dev, uint32_t k, uint32_t n, void *stream) {
  if (!weight_lpbq_dev || !block_scale_dev || !expanded_dev)
    return fail(QH_STATUS_INVALID_ARGUMENT, "qh_w4_lpbq_expand_to_i8: NULL buffer");
  if (k == 0 || n == 0 || k % 32 || n % 32 || k > (1u << 20) || n > (1u << 20))
    return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_w4_lpbq_expand_to_i8: K=%u N=%u (need multiples of 32, <= 2^20)", k, n);
  if (reinterpret_cast<uintptr_t>(weight_lpbq_dev) % 4 || reinterpret_cast<uintptr_t>(expanded_dev) % 16)
    return fail(QH_STATUS_INVALID_ARGUMENT,
                "qh_w4_lpbq_expand_to_i8: codes must be 4-byte and the output 16-byte aligned");
  return launch_lpbq_expand(weight_lpbq_dev, block_scale_dev, expanded_dev, k, n, static_cast<hipStream_t>(stream));
}

qh_status qh_gdn_solve_f32(const float *A_dev, float *T_dev, uint32_t heads, uint32_t C, uint32_t precision,
                           void *stream) {
  if (A_dev == nullptr || T_dev == nullptr) return fail(QH_STATUS_INVALID_ARGUMENT, "qh_gdn_solve_f32: NULL buffer");
  if (heads == 0 || heads > (1u << 24)) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_gdn_solve_f32: bad heads=%u", heads);
  if (C < 16 || C > 256 || C % 16) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_gdn_solve_f32: C=%u (need 16..256, C%%16==0)", C);
  if (precision > QH_GDN_BF16) return fail(QH_STATUS_UNSUPPORTED, "qh_gdn_solve_f32: unknown precision %u", precision);
  if (reinterpret_cast<uintptr_t>(A_dev) % 16 || reinterpret_cast<uintptr_t>(T_dev) % 16)
    return fail(QH_STATUS_INVALID_ARGUMENT, "qh_gdn_solve_f32: buffers must be 16-byte aligned");
  return launch_gdn_solve_f32(A_dev, T_dev, static_cast<int>(heads), static_cast<int>(C), static_cast<int>(precision),
                              static_cast<hipStream_t>(stream));
}

qh_status qh_gdn_solve_u16(const uint16_t *A_dev, uint16_t *T_dev, uint32_t heads, uint32_t C, int32_t zpA, int32_t zpT,
                           float sA, float sT, uint32_t precision, void *stream) {
  if (A_dev == nullptr || T_dev == nullptr) return fail(QH_STATUS_INVALID_ARGUMENT, "qh_gdn_solve_u16: NULL buffer");
  if (heads == 0 || heads > (1u << 24)) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_gdn_solve_u16: bad heads=%u", heads);
  if (C < 16 || C > 256 || C % 16) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_gdn_solve_u16: C=%u (need 16..256, C%%16==0)", C);
  if (precision > QH_GDN_OP_MODEL)
    return fail(QH_STATUS_UNSUPPORTED, "qh_gdn_solve_u16: unknown precision %u", precision);
  if (zpA < 0 || zpA > 65535 || zpT < 0 || zpT > 65535)
    return fail(QH_STATUS_INVALID_ARGUMENT, "qh_gdn_solve_u16: zero points must be in [0, 65535]");
  if (!(sA > 0.0f) || !(sT > 0.0f)) return fail(QH_STATUS_INVALID_ARGUMENT, "qh_gdn_solve_u16: scales must be > 0");
  if (reinterpret_cast<uintptr_t>(A_dev) % 16 || reinterpret_cast<uintptr_t>(T_dev) % 16)
    return fail(QH_STATUS_INVALID_ARGUMENT, "qh_gdn_solve_u16: buffers must be 16-byte aligned");
  if (precision == QH_GDN_OP_MODEL) {
    if (C > 64) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_gdn_solve_u16: the op model takes C <= 64 (C=%u)", C);
    return launch_gdn_solve_op_model(A_dev, T_dev, static_cast<int>(heads), static_cast<int>(C), zpA, zpT, sA, sT,
                                     static_cast<hipStream_t>(stream));
  }
  return launch_gdn_solve_u16(A_dev, T_dev, static_cast<int>(heads), static_cast<int>(C), zpA, zpT, sA, sT,
                              static_cast<int>(precision), static_cast<hipStream_t>(stream));
}


qh_status qh_gdn_chunk_uw_ex(const uint16_t *k_dev, const uint16_t *v_dev, const float *g_dev, const float *beta_dev,
                             void *w_dev, void *u_dev, uint32_t batch, uint32_t tokens, uint32_t heads,
                             uint32_t head_dim, uint32_t chunk, uint32_t flags, uint32_t max_workgroups,
                             void *stream) {
  if (!k_dev || !v_dev || !g_dev || !beta_dev || !w_dev || !u_dev)
    return fail(QH_STATUS_INVALID_ARGUMENT, "qh_gdn_chunk_uw: NULL buffer");
  if (head_dim != 128) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_gdn_chunk_uw: head_dim=%u (need 128)", head_dim);
  if (chunk != 64 && chunk != 128 && chunk != 256)
    return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_gdn_chunk_uw: chunk=%u (need 64, 128 or 256)", chunk);
  if (batch == 0 || heads == 0 || tokens == 0 || tokens % chunk)
    return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_gdn_chunk_uw: batch=%u tokens=%u heads=%u (tokens %% chunk == 0)",
                batch, tokens, heads);
  if (static_cast<uint64_t>(batch) * tokens * heads > (1ull << 31) / 128)
    return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_gdn_chunk_uw: batch * tokens * heads too large");
  if (flags & ~static_cast<uint32_t>(QH_GDN_W_DECAY | QH_GDN_OUT_F32))
    return fail(QH_STATUS_UNSUPPORTED, "qh_gdn_chunk_uw: unknown flags 0x%x", flags);
  const uintptr_t al = reinterpret_cast<uintptr_t>(k_dev) | reinterpret_cast<uintptr_t>(v_dev) |
                       reinterpret_cast<uintptr_t>(w_dev) | reinterpret_cast<uintptr_t>(u_dev);
  if (al % 16) return fail(QH_STATUS_INVALID_ARGUMENT, "qh_gdn_chunk_uw: k, v, w, u must be 16-byte aligned");
  if (max_workgroups > (1u << 24))
    return fail(QH_STATUS_INVALID_ARGUMENT, "qh_gdn_chunk_uw: max_workgroups=%u (0 = device-resident grid)",
                max_workgroups);
  return launch_gdn_chunk_uw(k_dev, v_dev, g_dev, beta_dev, w_dev, u_dev, static_cast<int>(batch),
                             static_cast<int>(tokens), static_cast<int>(heads), static_cast<int>(chunk),
                             static_cast<int>(flags), static_cast<int>(max_workgroups),
                             static_cast<hipStream_t>(stream));
}

qh_status qh_gdn_chunk_uw(const uint16_t *k_dev, const uint16_t *v_dev, const float *g_dev, const float *beta_dev,
                          void *w_dev, void *u_dev, uint32_t batch, uint32_t tokens, uint32_t heads,
                          uint32_t head_dim, uint32_t chunk, uint32_t flags, void *stream) {
  return qh_gdn_chunk_uw_ex(k_dev, v_dev, g_dev, beta_dev, w_dev, u_dev, batch, tokens, heads, head_dim, chunk, flags,
                            0, stream);
}

qh_status qh_gdn_chunk_state(const uint16_t *q_dev, const uint16_t *k_dev, const float *g_dev, const void *w_dev,
                             const void *u_dev, const float *s_in_dev, float *s_out_dev, void *o_dev, uint32_t batch,
                             uint32_t tokens, uint32_t heads, uint32_t head_dim, uint32_t chunk, uint32_t flags,
                             uint32_t precision, void *stream) {
  if (!q_dev || !k_dev || !g_dev || !w_dev || !u_dev || !s_out_dev || !o_dev)
    return fail(QH_STATUS_INVALID_ARGUMENT, "qh_gdn_chunk_state: NULL buffer");
  if (head_dim != 128) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_gdn_chunk_state: head_dim=%u (need 128)", head_dim);
  if (chunk != 64) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_gdn_chunk_state: chunk=%u (need 64)", chunk);
  if (batch == 0 || heads == 0 || tokens == 0 || tokens % 64)
    return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_gdn_chunk_state: batch=%u tokens=%u heads=%u (tokens %% 64 == 0)",
                batch, tokens, heads);
  if (static_cast<uint64_t>(batch) * tokens * heads > (1ull << 31) / 128 ||
      static_cast<uint64_t>(batch) * heads > (1u << 24))
    return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_gdn_chunk_state: batch * tokens * heads too large");
  if (flags & ~static_cast<uint32_t>(QH_GDN_OUT_F32 | QH_GDN_WU_F32))
    return fail(QH_STATUS_UNSUPPORTED, "qh_gdn_chunk_state: unknown flags 0x%x", flags);
  if (precision > QH_GDN_BF16) return fail(QH_STATUS_UNSUPPORTED, "qh_gdn_chunk_state: unknown precision %u", precision);
  if (s_in_dev != nullptr && s_in_dev == s_out_dev)
    return fail(QH_STATUS_INVALID_ARGUMENT, "qh_gdn_chunk_state: s_out_dev aliases s_in_dev");
  const uintptr_t al = reinterpret_cast<uintptr_t>(q_dev) | reinterpret_cast<uintptr_t>(k_dev) |
                       reinterpret_cast<uintptr_t>(w_dev) | reinterpret_cast<uintptr_t>(u_dev) |
                       reinterpret_cast<uintptr_t>(o_dev) | reinterpret_cast<uintptr_t>(s_out_dev) |
                       reinterpret_cast<uintptr_t>(s_in_dev);
  if (al % 16) return fail(QH_STATUS_INVALID_ARGUMENT, "qh_gdn_chunk_state: buffers must be 16-byte aligned");
  return launch_gdn_chunk_state(q_dev, k_dev, g_dev, w_dev, u_dev, s_in_dev, s_out_dev, o_dev, static_cast<int>(batch),
                                static_cast<int>(tokens), static_cast<int>(heads), static_cast<int>(precision),
                                (flags & QH_GDN_WU_F32) != 0, (flags & QH_GDN_OUT_F32) != 0,
                                static_cast<hipStream_t>(stream));
}

}  // extern "C"
