// Internal helpers shared by the gh_oracle translation units (test infrastructure).
#ifndef GHO_INTERNAL_H
#define GHO_INTERNAL_H
#include <stddef.h>
#include <stdint.h>

#include <functional>

namespace gho {
enum : uint32_t { FMT_F32 = 0, FMT_F16 = 1, FMT_Q4_K = 12, FMT_Q6_K = 14 };

int threads();
// for_units(len, stride, f): f(first_unit, start_elem, end_elem) per disjoint chunk.
void for_units(size_t len, size_t stride, const std::function<void(size_t, size_t, size_t)>& f);

float f16_to_f32(uint16_t h);
uint16_t f32_to_f16(float f);
void f16_slice_to_f32(const uint16_t* src, float* dst, size_t n);
void f32_slice_to_f16(const float* src, uint16_t* dst, size_t n);
void scale_min(const uint8_t* sc12, uint32_t j, uint32_t* sc, uint32_t* mn);
int dequant_row(uint32_t format, const uint8_t* bytes, size_t row, size_t in_dim, float* out);
size_t block_len(uint32_t format);
}  // namespace gho
#endif
