/* rns8 ABI basics for the MI355X implementation.
 *
 * Every public enum is stored in 32 bits. In C++ the enums carry an explicit
 * uint32_t base so that any 32-bit value received from a C or FFI caller can
 * be range-checked without undefined behaviour. C callers must use the normal
 * 32-bit enum ABI of their platform (no -fshort-enums).
 *
 * Layout contract: /root/reference include/rns8/abi.h:1-17 (same macro name
 * and meaning, so headers written against either library compile unchanged).
 */
#ifndef RNS8_ABI_H
#define RNS8_ABI_H

#include <stdint.h>

#ifdef __cplusplus
#define RNS8_ENUM_BASE : uint32_t
#else
#define RNS8_ENUM_BASE
#endif

#endif /* RNS8_ABI_H */
