#include "params.hpp"
namespace mote {
size_t decode_workspace_bytes(const mote_relation_decode_args*) { return 0; }
int launch_decode(const mote_relation_decode_args*, hipStream_t) { return set_error(MOTE_ERR_ARGUMENT, "relation_decode: not built"); }
}
