// tbe_internal.h — helpers shared by the HIP sources of libtbe_hip.so (not part
// of the C ABI).
#ifndef TBE_INTERNAL_H
#define TBE_INTERNAL_H

#include <stdint.h>

namespace tbe {

// Record a failure message for tbe_last_error() on this thread and return `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clear the message at the start of an entry point.
void clear_error();

}  // namespace tbe

#endif  // TBE_INTERNAL_H
