/* Byte-plane split/merge in plain C -- test infrastructure only.
 *
 * Restates formats/packed.py:49-50 (lo = raw[0::2], hi = raw[1::2]) and
 * formats/packed.py:376-378 (raw[0::2] = lo; raw[1::2] = hi) for little-endian
 * 16-bit elements.  Built by oracle/Makefile into liboracle_byteplane.so and
 * used by the tests and the bench's CPU baseline; never by the product.
 */
#include <stddef.h>
#include <stdint.h>

void oracle_byteplane_split(const uint16_t* src, uint8_t* lo, uint8_t* hi, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const uint16_t e = src[i];
    lo[i] = (uint8_t)(e & 0xffu);
    hi[i] = (uint8_t)(e >> 8);
  }
}

void oracle_byteplane_merge(const uint8_t* lo, const uint8_t* hi, uint16_t* dst, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    dst[i] = (uint16_t)((uint16_t)lo[i] | ((uint16_t)hi[i] << 8));
  }
}
