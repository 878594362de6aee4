// fp16x2 pair kernels: a call's RoPE and plain head-pair launch groups in one launch.
#include "restore_fast.h"

namespace rch {

PairFn pick_pair_fp16x2(int ks0, int ks1, int out_dtype, int* chosen0, int* chosen1) {
    return pick_pair<RCH_PREC_FP16X2>(ks0, ks1, out_dtype, chosen0, chosen1);
}

}  // namespace rch
