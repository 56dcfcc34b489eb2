// Work descriptors shared by the grouped expert kernels: a tile is a run of up to kExl3TileRows consecutive
// pair rows that all belong to one expert. Same struct and constant as the reference
// (src/kernels/exl3_moe.hpp:23-27); the EXL3 trellis kernels of that header are a different quantization
// format and are not part of this library.
#pragma once

namespace unholy::kernels {

constexpr int kExl3TileRows = 128;
struct Exl3Tile {
  int expert, row0, rows;
};

}  // namespace unholy::kernels
