// Decode-kernel instantiations for query type BF16 and FP8 E4M3 caches (paged
// 5-D layout, head sizes that are multiples of 16, every block size).  One
// translation unit per type pair keeps the kernel matrix compiling in
// parallel.
#include "paged_decode_impl.h"

namespace pkv {
template hipError_t launch_decode_typed<BF16, FP8>(const DecodeParams&, int, int, hipStream_t, bool*);
}  // namespace pkv
