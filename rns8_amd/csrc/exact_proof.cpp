// Exact-wide proofs: host side of the device proofs (see exact_proof.hpp).
#include "exact_proof.hpp"

#include "exact_range.hpp"
#include "kernels.hpp"

namespace rns8x {

namespace {

using Kind = rns8_matrix::ProofKind;

I512 from_words(const uint64_t* w) {
  I512 r;
  for (int i = 0; i < 4; ++i) r.w[i] = w[i];
  return r;
}

// the axis kind a current (not lazy) proof hands to the product kernels
uint32_t axis_kind(const rns8_matrix& m) {
  return static_cast<uint32_t>(m.proof_kind == Kind::Native    ? xa::AxisKind::Native
                               : m.proof_kind == Kind::Carried ? xa::AxisKind::Carried
                                                               : xa::AxisKind::Uniform);
}

rns8_status read_words(const uint64_t* src, hipStream_t stream, uint64_t (&w)[4]) {
  if (hipMemcpyAsync(w, src, sizeof(w), hipMemcpyDeviceToHost, stream) != hipSuccess ||
      hipStreamSynchronize(stream) != hipSuccess)
    return RNS8_BACKEND_FAILURE;
  return RNS8_SUCCESS;
}

}  // namespace

rns8_status prove_native(const rns8_matrix& m, const void* src, int64_t ld, bool is_signed, hipStream_t stream) {
  const uint32_t t = m.proof_set ^ 1u;
  return launch_native_axes(src, m.desc.rows, m.desc.cols, ld, is_signed, m.row_partials(), m.col_partials(),
                            m.proof_rows(t), m.proof_cols(t), m.proof_words(t), stream) == hipSuccess
             ? RNS8_SUCCESS
             : RNS8_BACKEND_FAILURE;
}

rns8_status read_free_bound(const rns8_matrix& m, hipStream_t stream, I512& out) {
  uint64_t w[4];
  const rns8_status st = read_words(m.proof_words(m.proof_set ^ 1u), stream, w);
  if (st == RNS8_SUCCESS) out = from_words(w);
  return st;
}

rns8_status commit_native_proof(rns8_matrix& m, const I512& bound, bool pending, hipStream_t stream) {
  if (hipEventRecord(m.proof_event, stream) != hipSuccess) return RNS8_BACKEND_FAILURE;
  m.proof_set ^= 1u;
  m.proof_kind = Kind::Native;
  m.exact_max = bound;
  m.exact_pending = pending;
  m.exact_prefix = m.prefix;
  return RNS8_SUCCESS;
}

rns8_status materialize_proof(const rns8_matrix& m, hipStream_t stream) {
  if (m.proof_kind != Kind::Lazy) return RNS8_SUCCESS;
  const uint32_t s = m.proof_set, t = s ^ 1u;
  const bool uniform = m.lazy_rows == static_cast<uint32_t>(xa::AxisKind::Uniform) &&
                       m.lazy_cols == static_cast<uint32_t>(xa::AxisKind::Uniform);
  if (launch_product_axes(m.proof_rows(s), m.lazy_rows, m.proof_cols(s), m.lazy_cols, m.proof_words(s),
                          m.proof_words(s) + 4, m.desc.rows, m.desc.cols, m.lazy_k, m.proof_rows(t),
                          m.proof_cols(t), m.proof_words(t), stream) != hipSuccess ||
      hipEventRecord(m.proof_event, stream) != hipSuccess)
    return RNS8_BACKEND_FAILURE;
  m.proof_set = t;
  m.proof_kind = uniform ? Kind::Uniform : Kind::Carried;
  return RNS8_SUCCESS;
}

rns8_status resolve_exact_proof(const rns8_matrix& m, hipStream_t stream) {
  if (!m.exact_pending) return RNS8_SUCCESS;
  if (hipSetDevice(m.device_id) != hipSuccess) return RNS8_BACKEND_FAILURE;
  if (m.proof_kind == Kind::Lazy) {
    if (hipStreamWaitEvent(stream, m.proof_event, 0) != hipSuccess) return RNS8_BACKEND_FAILURE;
    const rns8_status st = materialize_proof(m, stream);
    if (st != RNS8_SUCCESS) return st;
  }
  uint64_t w[4];
  if (hipEventSynchronize(m.proof_event) != hipSuccess ||
      hipMemcpy(w, m.proof_words(m.proof_set), sizeof(w), hipMemcpyDeviceToHost) != hipSuccess)
    return RNS8_BACKEND_FAILURE;
  m.exact_max = from_words(w);
  m.exact_pending = false;
  return RNS8_SUCCESS;
}

rns8_status exact_gemm_admit(const rns8_plan& plan, const rns8_matrix& A, const rns8_matrix& B,
                             const rns8_matrix& C, hipStream_t stream, ExactAdmission& out) {
  if (A.exact_prefix < plan.prefix || B.exact_prefix < plan.prefix) return RNS8_RANGE_ERROR;
  const I512 k = I512::from_u64(static_cast<uint64_t>(plan.desc.k));
  out.refined = false;
  out.bound = k * A.exact_max * B.exact_max;
  // the reference's bound is at most k maxA maxB (exact_range.hpp:113)
  if (exact_range_fits(plan.desc.semantics, out.bound, plan.product)) return RNS8_SUCCESS;
  rns8_status st = materialize_proof(A, stream);
  if (st == RNS8_SUCCESS) st = materialize_proof(B, stream);
  if (st != RNS8_SUCCESS) return st;
  const uint32_t t = C.proof_set ^ 1u;
  if (launch_product_axes(A.proof_rows(A.proof_set), axis_kind(A), B.proof_cols(B.proof_set), axis_kind(B),
                          A.proof_words(A.proof_set), B.proof_words(B.proof_set), plan.desc.m, plan.desc.n,
                          static_cast<uint64_t>(plan.desc.k), C.proof_rows(t), C.proof_cols(t), C.proof_words(t),
                          stream) != hipSuccess)
    return RNS8_BACKEND_FAILURE;
  uint64_t w[4];
  st = read_words(C.proof_words(t), stream, w);
  if (st != RNS8_SUCCESS) return st;
  out.refined = true;
  out.bound = from_words(w);
  return exact_range_fits(plan.desc.semantics, out.bound, plan.product) ? RNS8_SUCCESS : RNS8_RANGE_ERROR;
}

rns8_status commit_exact_proof(rns8_matrix& C, const rns8_matrix& A, const rns8_matrix& B, const rns8_plan& plan,
                               const ExactAdmission& adm, hipStream_t stream) {
  const uint32_t t = C.proof_set ^ 1u;
  if (adm.refined) {
    // the summaries are already in the free set
    C.proof_kind = axis_kind(A) == static_cast<uint32_t>(xa::AxisKind::Uniform) &&
                           axis_kind(B) == static_cast<uint32_t>(xa::AxisKind::Uniform)
                       ? Kind::Uniform
                       : Kind::Carried;
    C.exact_pending = false;
  } else {
    rns8_status st = materialize_proof(A, stream);
    if (st == RNS8_SUCCESS) st = materialize_proof(B, stream);
    if (st != RNS8_SUCCESS) return st;
    const uint32_t ak = axis_kind(A), bk = axis_kind(B);
    const bool a_axes = ak != static_cast<uint32_t>(xa::AxisKind::Uniform);
    const bool b_axes = bk != static_cast<uint32_t>(xa::AxisKind::Uniform);
    if (launch_proof_snapshot(a_axes ? A.proof_rows(A.proof_set) : nullptr,
                              b_axes ? B.proof_cols(B.proof_set) : nullptr, A.proof_words(A.proof_set),
                              B.proof_words(B.proof_set), a_axes ? plan.desc.m : 0, b_axes ? plan.desc.n : 0,
                              C.proof_rows(t), C.proof_cols(t), C.proof_words(t), stream) != hipSuccess)
      return RNS8_BACKEND_FAILURE;
    C.proof_kind = Kind::Lazy;
    C.lazy_rows = ak;
    C.lazy_cols = bk;
    C.lazy_k = static_cast<uint64_t>(plan.desc.k);
    C.exact_pending = true;
  }
  if (hipEventRecord(C.proof_event, stream) != hipSuccess) return RNS8_BACKEND_FAILURE;
  C.proof_set = t;
  C.exact_max = adm.bound;
  C.exact_prefix = plan.prefix;
  return RNS8_SUCCESS;
}

}  // namespace rns8x
