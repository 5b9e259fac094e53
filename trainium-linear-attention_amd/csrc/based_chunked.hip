// Chunked recurrent BASED attention (kernel under construction).
#include "../../include/based_la.h"
#include "la_internal.hpp"

namespace la {
size_t chunked_workspace_bytes(int, int, int, int, int) { return (size_t)-1; }
int launch_based_chunked(const ChunkedArgs&, hipStream_t) { return LA_ERR_UNSUPPORTED_DIM; }
}  // namespace la
