// qmm_layout.h - host-side placement of GGUF blocks in the weight image.
#pragma once

#include "qmm_internal.h"

namespace qmm {

// global tile of global row R (R = mat * M + m); rows [r0, r1) of tile T
int64_t tile_of_row(const ImageShape & s, int64_t R);
void tile_rows(const ImageShape & s, int64_t T, int64_t * r0, int64_t * r1);

// Blocks [b0, b0 + nb) of the tensor (global block index: row-major over all
// matrices) between their GGUF bytes and `img`, the image bytes of the global
// tiles starting at T0 (every touched tile must be inside img).
void pack_blocks(const TypeLayout & L, const ImageShape & s, const uint8_t * src, int64_t b0, int64_t nb,
                 uint8_t * img, int64_t T0);
void unpack_blocks(const TypeLayout & L, const ImageShape & s, const uint8_t * img, int64_t T0, int64_t b0, int64_t nb,
                   uint8_t * dst);
// zero the padding blocks of global row R's last group (Q4_0 / Q8_0 rows
// whose length is not a multiple of 256)
void zero_row_padding(const TypeLayout & L, const ImageShape & s, int64_t R, uint8_t * img, int64_t T0);

}  // namespace qmm
