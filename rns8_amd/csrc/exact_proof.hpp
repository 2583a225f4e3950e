// Exact-wide admission and the proofs exact-wide matrices carry (reference
// src/core/exact_range.hpp:104-171, api_gemm.cpp:870-874, api_pack.cpp:47-65,
// api_export.cpp:42-47). The proofs live on the device (rns8_matrix's
// proof_device, kernels in exact_axes.hip); the host keeps a bound that the
// exact one never exceeds, decides on it while it passes, and otherwise
// computes the reference's refined bound on the device and reads it back.
#pragma once

#include <hip/hip_runtime_api.h>

#include "handles.hpp"

namespace rns8x {

// A pack's proof: the operand's native summaries into the matrix's free set
// (made current by commit_native_proof).
rns8_status prove_native(const rns8_matrix& m, const void* src, int64_t ld, bool is_signed, hipStream_t stream);
// Reads the free set's bound (max |x|) back; synchronizes the stream.
rns8_status read_free_bound(const rns8_matrix& m, hipStream_t stream, I512& out);
// Makes the free set current as a native proof; `bound` is exact or, when
// `pending`, a worst case of max |x|.
rns8_status commit_native_proof(rns8_matrix& m, const I512& bound, bool pending, hipStream_t stream);

// Computes a lazy proof's own summaries (a no-op for other proofs).
rns8_status materialize_proof(const rns8_matrix& m, hipStream_t stream);
// Makes exact_max exact: materializes a lazy proof on `stream` (after the
// proof's last writer) and reads the bound back.
rns8_status resolve_exact_proof(const rns8_matrix& m, hipStream_t stream);

// The admission of an exact-wide C = A x B (exact_range.hpp:147-157): the
// worst case k * A.exact_max * B.exact_max when it fits (C's proof is then
// lazy), otherwise the reference's refined bound computed on the device into
// C's free set and read back (the call synchronizes the stream).
struct ExactAdmission {
  bool refined = false;
  I512 bound;  // lazy: the worst case; refined: exact
};
rns8_status exact_gemm_admit(const rns8_plan& plan, const rns8_matrix& A, const rns8_matrix& B,
                             const rns8_matrix& C, hipStream_t stream, ExactAdmission& out);
// C's proof after its GEMM was launched on `stream` (exact_range.hpp:159-171).
rns8_status commit_exact_proof(rns8_matrix& C, const rns8_matrix& A, const rns8_matrix& B, const rns8_plan& plan,
                               const ExactAdmission& adm, hipStream_t stream);

}  // namespace rns8x
