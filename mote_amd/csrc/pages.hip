// Arena rows <-> prefix-store pages (mote/infer/prefix_cache.py:144-165) as strided DMA.
//
// The rows [r0, r0 + n) of one (layer, kind) plane of one sequence are H runs of n * D elements,
// capacity * D apart in the arena and page_rows * D apart in a page: exactly a 2-D copy, which the
// DMA engines do from pinned host memory without a staging buffer or a kernel. One call per plane
// (2 * n_layers per page segment).
#include "params.hpp"

namespace mote {

int launch_page_copy(const mote_page_copy_args* a, hipStream_t stream) {
  if (!a) return set_error(MOTE_ERR_ARGUMENT, "arena_page_copy: null args");
  if (a->planes < 0 || a->H <= 0 || a->D <= 0 || a->rows < 0 || (a->elem_bytes != 2 && a->elem_bytes != 4))
    return set_error(MOTE_ERR_SHAPE, "arena_page_copy: bad sizes");
  if (a->rows == 0 || a->planes == 0) return MOTE_OK;
  if (!a->arena || !a->page) return set_error(MOTE_ERR_ARGUMENT, "arena_page_copy: null pointer");
  if (a->arena_row0 < 0 || a->page_row0 < 0 || a->a_head < int64_t(a->D) || a->p_head < int64_t(a->D))
    return set_error(MOTE_ERR_ARGUMENT, "arena_page_copy: bad offsets or strides");
  const size_t eb = size_t(a->elem_bytes);
  const size_t width = size_t(a->rows) * a->D * eb;
  char* ar = reinterpret_cast<char*>(a->arena) + size_t(a->arena_row0) * a->D * eb;
  char* pg = reinterpret_cast<char*>(a->page) + size_t(a->page_row0) * a->D * eb;
  for (int i = 0; i < a->planes; ++i) {
    char* ap = ar + size_t(i) * a->a_plane * eb;
    char* pp = pg + size_t(i) * a->p_plane * eb;
    const hipError_t e = a->to_page
        ? hipMemcpy2DAsync(pp, size_t(a->p_head) * eb, ap, size_t(a->a_head) * eb, width, a->H, hipMemcpyDefault, stream)
        : hipMemcpy2DAsync(ap, size_t(a->a_head) * eb, pp, size_t(a->p_head) * eb, width, a->H, hipMemcpyDefault, stream);
    if (e != hipSuccess) return set_error(MOTE_ERR_LAUNCH, "arena_page_copy: hipMemcpy2DAsync: %s", hipGetErrorString(e));
  }
  return MOTE_OK;
}

}  // namespace mote
