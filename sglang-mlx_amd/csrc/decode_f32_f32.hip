// Decode-kernel instantiations for query type F32 and cache type F32 (every
// supported head size and block size; paged layout).  One translation unit
// per type pair keeps the kernel matrix compiling in parallel.
#include "paged_decode_impl.h"

namespace pkv {
template hipError_t launch_decode_typed<F32, F32>(const DecodeParams&, int, int, hipStream_t, bool*);
}  // namespace pkv
