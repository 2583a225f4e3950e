/* Modulus ladder queries. Constants and entry points follow reference
 * include/rns8/moduli.h:12-20. The ladder itself is
 * 256, 255, 253, 251, 247, 239, 233, 229, 227, 223, 217, 211, 199, 197,
 * 193, 191, 181, 179, 173, 167, 163, 157, 151, 149, 139, 137, 131, 127
 * (reference src/core/internal.hpp:328-330); at most the first 20 are used. */
#ifndef RNS8_MODULI_H
#define RNS8_MODULI_H

#include <stdint.h>

#include "rns8/status.h"

#ifdef __cplusplus
extern "C" {
#endif

#define RNS8_DEFAULT_MODULUS_COUNT 28u
#define RNS8_DEFAULT_BOUNDED_PREFIX 9u
#define RNS8_MAX_SUPPORTED_PREFIX 20u
/* 65536 * 128 * 128 + 128 fits in int32: the longest K run accumulated in
 * int32 before a modular reduction. */
#define RNS8_SAFE_INT32_K_BLOCK 65536u

/* reference moduli.h:17 */
RNS8_API uint32_t rns8_default_modulus_count(void);
/* reference moduli.h:18; returns 0 for an index past the ladder */
RNS8_API uint16_t rns8_default_modulus(uint32_t index);
/* reference moduli.h:19; sum of log2(m_i) over the prefix, 0.0 if invalid */
RNS8_API double rns8_prefix_range_bits(uint32_t prefix);
/* reference moduli.h:20; SUCCESS when the ladder is pairwise coprime */
RNS8_API rns8_status rns8_validate_default_moduli(void);

#ifdef __cplusplus
}
#endif

#endif /* RNS8_MODULI_H */
