// fp16 variants of the fused restore kernel (one translation unit per precision).
#include "restore_fast.h"

namespace rch {

RestoreVariant pick_restore_fp16(int source_kind, int ks) { return pick_source<RCH_PREC_FP16>(source_kind, ks); }

FastFn pick_fast_fp16(int ks, bool rope, int out_dtype, int shape, int* chosen) {
    return pick_fast<RCH_PREC_FP16>(ks, rope, out_dtype, shape, chosen);
}


}  // namespace rch
