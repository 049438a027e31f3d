// Decode-kernel instantiations for query type F16 and cache type F16 (every
// supported head size and block size).  One translation unit per type pair
// keeps the kernel matrix compiling in parallel.
#include "paged_decode_impl.h"

namespace pkv {
template hipError_t launch_decode_typed<F16, F16>(const DecodeParams&, int, int, hipStream_t, bool*);
}  // namespace pkv
