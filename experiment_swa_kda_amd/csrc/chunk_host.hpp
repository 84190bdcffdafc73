// Host helpers shared by the chunked forward and backward translation units.
#pragma once

#include "chunk_layout.hpp"
#include "kda_host.hpp"

namespace kda {

int validate_problem(const kda_chunk_problem* p, const char* who);
ChunkGeom make_geom(const kda_chunk_problem* p);
int launch_chunk_prep(const kda_chunk_problem* p, const ChunkGeom& g, const Regions& ws,
                      hipStream_t stream);

}  // namespace kda
