// dec_m0.hip -- decode-shaped flash attention instantiations without a mask.
#include "fa_decode_inst.h"

namespace cvattn {
CVATTN_DECODE_PICK(fa_pick_decode_m0, false)
} // namespace cvattn
