#include "params.hpp"
namespace mote {
size_t bwd_workspace_bytes(const mote_relation_bwd_args*) { return 0; }
int launch_bwd(const mote_relation_bwd_args*, hipStream_t) { return set_error(MOTE_ERR_ARGUMENT, "relation_bwd: not built"); }
}
