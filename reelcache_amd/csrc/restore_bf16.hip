// bf16 variants of the fused restore kernel (one translation unit per precision).
#include "restore_kernel.h"

namespace rch {

RestoreVariant pick_restore_bf16(int source_kind, int ks) { return pick_source<RCH_PREC_BF16>(source_kind, ks); }

}  // namespace rch
