// C entry points over the reference's own GGUF dequantizer (csrc/artlite/dequant.{h,cpp} of the reference, compiled
// from its sources by oracle/Makefile into oracle/_ref/): the oracle's cross-check of its numpy restatement.
// Test infrastructure only.
#include <cstddef>
#include <cstdint>
#include <exception>

#include "artlite/dequant.h"

extern "C" int ref_dequant_supported(const char* qtype) { return artlite::dequant_supported(qtype) ? 1 : 0; }

extern "C" int ref_dequant_rows(const char* qtype, const uint8_t* raw, size_t n, size_t row_bytes, size_t cols,
                                float* out) {
  try {
    artlite::dequant_rows(qtype, raw, n, row_bytes, cols, out);
    return 0;
  } catch (const std::exception&) {
    return 1;
  }
}
