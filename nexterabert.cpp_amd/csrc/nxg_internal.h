// nxg_internal.h -- declarations shared by the host and device halves of libnxg.
#ifndef NXG_INTERNAL_H
#define NXG_INTERNAL_H

#include <stddef.h>
#include <stdint.h>

// Copies rows of n_in int8 values (row-major) into 16-row x 64-input fragment
// tiles: byte (r, k) goes to ((r/16)*KS + k/64)*1024 + ((r%16) + 16*((k%64)/16))*16 + k%16.
// `tiled` must be zero-filled and hold ceil(n_rows/16)*16 * KS*64 bytes. n_in % 16 == 0.
void nxg_tile_rows(const int8_t * rows, int n_rows, int n_in, int KS, int8_t * tiled);

// Records the message returned by nxg_last_error() on this thread.
void nxg_set_error(const char * msg);

#endif
