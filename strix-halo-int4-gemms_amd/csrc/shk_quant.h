// Device fake quantization and int4 packing (k_quant.hip), shared with the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace shk {

struct QuantArgs {
  const void* x;   // source values, row pitch ld_x elements
  uint8_t* out;    // output, row pitch ld_out bytes
  long rows, cols, ld_x, ld_out;
  long out_rows, out_cols;  // output extent in rows and bytes
  float inv;       // the fp32 reciprocal of the scale
  int bits;        // 4 or 8
  int src;         // SHK_SRC_*
  int mode;        // SHK_QUANT_*
};

hipError_t launch_quantize(const QuantArgs& p, hipStream_t s);

}  // namespace shk
