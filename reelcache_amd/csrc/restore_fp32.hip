// fp32 variants of the fused restore kernel (one translation unit per precision).
#include "restore_kernel.h"

namespace rch {

RestoreVariant pick_restore_fp32(int source_kind, int ks) { return pick_source<RCH_PREC_FP32>(source_kind, ks); }

}  // namespace rch
