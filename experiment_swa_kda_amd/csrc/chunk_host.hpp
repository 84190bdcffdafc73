// Host helpers shared by the chunked forward and backward translation units.
#pragma once

#include "chunk_layout.hpp"
#include "kda_host.hpp"

namespace kda {

int validate_problem(const kda_chunk_problem* p, const char* who);
ChunkGeom make_geom(const kda_chunk_problem* p);
int launch_chunk_prep(const kda_chunk_problem* p, const ChunkGeom& g, const Regions& ws,
                      hipStream_t stream);

// Token-serial path for head dims other than 64 / 128 (generic.hip).
bool generic_dims(const kda_chunk_problem* p);
size_t generic_ws_bytes(const kda_chunk_problem* p);
size_t generic_sc_bytes(const kda_chunk_problem* p);
int generic_forward(const kda_chunk_problem* p, const void* q, const void* k, const void* v, const void* gate,
                    const void* beta_logits, const float* A_log, const float* dt_bias, const float* initial_state,
                    void* output, float* final_state, void* workspace, hipStream_t stream);
int generic_backward(const kda_chunk_problem* p, const void* q, const void* k, const void* v, const void* gate,
                     const void* beta_logits, const float* A_log, const float* dt_bias, const void* workspace,
                     const void* grad_output, const float* grad_final_state, void* dq, void* dk, void* dv,
                     void* dgate, void* dbeta_logits, float* dA_log, float* ddt_bias, float* dinitial_state,
                     void* scratch, hipStream_t stream);

// Zero-padded route (generic.hip): K, V <= 128 other than 64 / 128 run the chunked kernels
// at K, V rounded up to 64 or 128.
bool padded_route(const kda_chunk_problem* p);
size_t padded_ws_bytes(const kda_chunk_problem* p);
size_t padded_sc_bytes(const kda_chunk_problem* p);
int padded_forward(const kda_chunk_problem* p, const void* q, const void* k, const void* v, const void* gate,
                   const void* beta_logits, const float* A_log, const float* dt_bias, const float* initial_state,
                   void* output, float* final_state, void* workspace, hipStream_t stream);
int padded_backward(const kda_chunk_problem* p, const void* beta_logits, const float* A_log, const void* workspace,
                    const void* grad_output, const float* grad_final_state, void* dq, void* dk, void* dv,
                    void* dgate, void* dbeta_logits, float* dA_log, float* ddt_bias, float* dinitial_state,
                    void* scratch, hipStream_t stream);
int padded_status(const kda_chunk_problem* p, const void* scratch, hipStream_t stream);

constexpr size_t cmax_sz(size_t x, size_t y) { return x > y ? x : y; }

// Compute units of the current device (launch granularity of the chunk-parallel rounds and
// the fused launches' sizing); 0 if it cannot be queried.
inline int device_cu_count() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess) cached[dev] = n;
  }
  return cached[dev];
}

}  // namespace kda
