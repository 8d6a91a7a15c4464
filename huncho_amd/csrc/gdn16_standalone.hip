// gdn16_standalone.hip - the standalone chunked delta-rule recurrence, gdn_chunk16<T, false>
// (kernel in gdn16_kernel.hpp), in a translation unit of its own: the build compiles it with the
// max-memory-clause machine scheduler, which runs this instantiation 5-6 % faster at the Kev
// 64 x 512 shape while the fused layer kernel is 4-5 % faster with the default scheduler.
#include "gdn16_kernel.hpp"

int hk_launch_gdn16_standalone(int dtype16, const hk::GdnArgs* a, int n_seqs, hipStream_t stream) {
    const hk::GdnFusedArgs none{};
    return dtype16 == 1 ? launch16<hk::bf16, false>(a, &none, n_seqs, stream)
                        : launch16<hk::f16, false>(a, &none, n_seqs, stream);
}
