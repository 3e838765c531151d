// dec_m1_h1.hip -- decode-shaped flash attention instantiations: masked, one kv head per workgroup.
#include "fa_decode_inst.h"

namespace cvattn {
CVATTN_DECODE_PICK(fa_pick_decode_m1_h1, true, 1)
} // namespace cvattn
