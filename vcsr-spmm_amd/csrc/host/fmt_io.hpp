// fmt_io.hpp - VCSR format files (fmt_io.cpp) and the structural check a
// format must pass before the kernels may index with it.
#pragma once

#include <cstdint>
#include <string>

#include "core.hpp"

namespace vcsr {

// Throws Error(VCSR_EINVAL) unless v satisfies what the builders produce and
// the kernels rely on: consistent array sizes, group_ptr advancing by
// depth * bundle, rows in [-1, M), local columns inside their segment and
// inside [0, N), each lane's entries packed from depth 0, the lanes with
// entries a prefix of each group, and segment_group_start matching the
// groups' segment bases.
void validate_vcsr(const Vcsr& v);

void save_vcsr(const Vcsr& v, int32_t tile_rows, bool tile_fixed, const std::string& path);
// Reads and validates a file written by save_vcsr (VCSR_EIO when it cannot
// be read, VCSR_EINVAL when its contents are not a valid format).
Vcsr load_vcsr(const std::string& path, int32_t* tile_rows, bool* tile_fixed);

}  // namespace vcsr
