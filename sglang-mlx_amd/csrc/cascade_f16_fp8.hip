// Cascade (shared-prefix) decode instantiations for query type F16 and cache
// type FP8 (head sizes 64 and 128, every block size).  One translation unit
// per type pair keeps the kernels compiling in parallel.
#include "cascade_impl.h"

namespace pkv {
template hipError_t launch_cascade_typed<F16, FP8>(const DecodeParams&, const CascadeParams&, int, int, hipStream_t,
                                                 bool*);
}  // namespace pkv
