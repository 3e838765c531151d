// dec_m0_h1.hip -- decode-shaped flash attention instantiations: unmasked, one kv head per workgroup.
#include "fa_decode_inst.h"

namespace cvattn {
CVATTN_DECODE_PICK(fa_pick_decode_m0_h1, false, 1)
} // namespace cvattn
