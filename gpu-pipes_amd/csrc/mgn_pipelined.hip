// Stage-chained MGN MLP (workgroup stages linked by L2 ring queues).
#include "gp_host.hpp"
#include "../../include/gpipes.h"

namespace gp {
int mgn_pipelined_run(const MgnArgs&, int, int, hipStream_t) {
  return fail(GP_ERR_INVALID_ARG, "GP_IMPL_PIPELINED is not built in this version");
}
}  // namespace gp
