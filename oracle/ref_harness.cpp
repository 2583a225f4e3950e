// Harness exposing the reference's own header-only arithmetic through a C ABI
// so tests can pin the oracle against it. TEST INFRASTRUCTURE ONLY.
//
// Compiled by oracle/Makefile (target `ref`) directly against the sources where
// they lie under /root/reference/src/backend_common/ (finite_u8_reducer.hpp,
// residue_dot.hpp). Those headers are plain C++17 without HIP; no stand-in
// header, library or macro is supplied. The result goes to oracle/_ref/ only
// and is never part of the product library.
#include <cstdint>

#include "finite_u8_reducer.hpp"
#include "residue_dot.hpp"

namespace fin = rns8::detail::finite_u8;

extern "C" {

// finite_u8_reducer.hpp:145-165
int8_t ref_reduce_to_centered_i32(int32_t value, uint32_t modulus) {
  return fin::reduce_to_centered_i32(value, modulus, fin::modulus_reciprocal_u32(modulus));
}

// finite_u8_reducer.hpp:167-187
int8_t ref_reduce_to_centered_accelerator_i32(int32_t value, uint32_t modulus) {
  return fin::reduce_to_centered_accelerator_i32(value, modulus, fin::modulus_reciprocal_u32(modulus));
}

// finite_u8_reducer.hpp:282-293
int8_t ref_center_u8(uint8_t value, uint32_t modulus) { return fin::center_u8(value, modulus); }

// finite_u8_reducer.hpp:308-311
uint32_t ref_canonical_from_centered(int8_t residue, uint32_t modulus) {
  return fin::canonical_from_centered(residue, modulus);
}

// residue_dot.hpp:21-38
int8_t ref_centered_residue_dot(const int8_t* a, const int8_t* b, int64_t k, int64_t b_stride, uint32_t modulus) {
  return rns8::detail::centered_residue_dot(a, b, k, b_stride, modulus);
}

// Batch helper: reduce `count` int32 values (the reference reducer per value).
void ref_reduce_many(const int32_t* values, int64_t count, uint32_t modulus, int8_t* out) {
  const uint32_t reciprocal = fin::modulus_reciprocal_u32(modulus);
  for (int64_t i = 0; i < count; ++i) out[i] = fin::reduce_to_centered_i32(values[i], modulus, reciprocal);
}

}  // extern "C"
