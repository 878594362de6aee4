// Variants of the basis-stationary stream kernel (restore_stream.h), in their own translation unit.
#include "restore_stream.h"

namespace rch {

StreamFn pick_stream_fp16x2(int ks, int rope, int out_dtype, int* chosen) {
    switch (rope) {
        case kRopeNone: return stream_out<kRopeNone>(ks, out_dtype, chosen);
        case kRopeSections: return stream_out<kRopeSections>(ks, out_dtype, chosen);
        case kRopeDense: return stream_out<kRopeDense>(ks, out_dtype, chosen);
        default: *chosen = 0; return nullptr;
    }
}

}  // namespace rch
