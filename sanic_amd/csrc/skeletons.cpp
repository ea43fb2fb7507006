// Hand-written CDNA4 skeletons, chosen from the structure of a stage's carrier and leaves.
#include "emit.h"

namespace sanic {

bool lower_skeleton(const sanic_program_desc*, int, int64_t&, LoweredStage&) { return false; }
bool lower_pointwise_skeleton(const sanic_program_desc*, int, int64_t&, LoweredStage&) { return false; }

}  // namespace sanic
