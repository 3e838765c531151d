// dec_m1.hip -- decode-shaped flash attention instantiations with a mask.
#include "fa_decode_inst.h"

namespace cvattn {
CVATTN_DECODE_PICK(fa_pick_decode_m1, true)
} // namespace cvattn
