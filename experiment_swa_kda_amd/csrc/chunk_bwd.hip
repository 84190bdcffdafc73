// Chunked backward (placeholder until the kernels land).
#include "chunk_host.hpp"

extern "C" int kda_chunk_backward(const kda_chunk_problem* p, const void*, const void*,
                                  const void*, const void*, const void*, const float*,
                                  const float*, const float*, const void*, const void*,
                                  const float*, void*, void*, void*, void*, void*, float*,
                                  float*, float*, void*, hipStream_t) {
  (void)p;
  return kda::set_error(KDA_ERR_INVALID, "chunk_backward: not implemented");
}
