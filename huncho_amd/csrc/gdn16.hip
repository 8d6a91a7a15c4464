// gdn16.hip - the fused Gated DeltaNet layer instantiations of gdn_chunk16 (the kernel is in
// gdn16_kernel.hpp) and the 16-bit delta-rule launcher. The standalone recurrence is
// instantiated in gdn16_standalone.hip, which the build compiles with its own machine
// scheduling strategy.
#include "gdn16_kernel.hpp"

int hk_launch_gdn16_standalone(int dtype16, const hk::GdnArgs* a, int n_seqs, hipStream_t stream);

// dtype16: 1 = bf16, 2 = fp16
extern "C" int hk_launch_gdn16(int dtype16, int fused, const hk::GdnArgs* a, const hk::GdnFusedArgs* fa, int n_seqs,
                               hipStream_t stream) {
    if (!fused) return hk_launch_gdn16_standalone(dtype16, a, n_seqs, stream);
    if (!fa) return HK_ERR_INVALID;
    return dtype16 == 1 ? launch16<hk::bf16, true>(a, fa, n_seqs, stream) : launch16<hk::f16, true>(a, fa, n_seqs, stream);
}
