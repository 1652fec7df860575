/* Tail-safe tile loaders for packed GLINT planes (host C/C++).
 * Reference: include/glint_htile_load.h:11-32 (same names and results).
 *
 * glint_packed_tile_byte: the packed byte holding elements (row, k) and (row, k+1) of a
 *   [rows, K] matrix packed along K, for any K parity; a nibble whose row >= rows or
 *   whose column >= K reads as 0.
 * glint_x_tile_element: x[row, k], or 0 outside [rows, K). */
#ifndef GLINT_HTILE_LOAD_H_
#define GLINT_HTILE_LOAD_H_
#include <stdint.h>

static inline uint8_t glint_nibble_at(const uint8_t *packed, int64_t i) {
    return (uint8_t)((packed[i >> 1] >> ((i & 1) * 4)) & 15u);
}

static inline uint8_t glint_packed_tile_byte(const uint8_t *packed, int row, int rows, int K, int k) {
    if (row >= rows)
        return 0;
    const int64_t base = (int64_t)row * K;
    const uint8_t lo = k < K ? glint_nibble_at(packed, base + k) : 0;
    const uint8_t hi = k + 1 < K ? glint_nibble_at(packed, base + k + 1) : 0;
    return (uint8_t)(lo | (hi << 4));
}

#define GLINT_X_TILE_ELEMENT(x, row, rows, K, k) \
    (((row) < (rows) && (k) < (K)) ? (x)[(int64_t)(row) * (K) + (k)] : 0)

#ifdef __cplusplus
template <typename T>
static inline T glint_x_tile_element(const T *x, int row, int rows, int K, int k) {
    return row < rows && k < K ? x[(int64_t)row * K + k] : T(0);
}
#endif
#endif
