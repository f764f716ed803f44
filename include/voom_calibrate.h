/*
 * voom_calibrate.h - C ABI of libvoom_calibrate.so: probe kernels that bench.py
 * times to give floors for the kernels of libvoom_hip.so (a plain streaming
 * read, a row gather, the MLA latent kernel's data movement).  Not part of the
 * paged-KV path and not loaded by it; no counterpart in the reference.
 * Conventions (pointers, streams, return codes, voom_last_error) are those of
 * voom_hip.h; the library links against libvoom_hip.so.
 */
#ifndef VOOM_CALIBRATE_H
#define VOOM_CALIBRATE_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------------
 * One launch that reads
 * n_bytes of device memory (16-byte aligned) with `workgroups` workgroups of
 * 256; sink[w] ^= the XOR of the words workgroup w read.  bench.py times
 * it to give the floor of a single launch streaming a buffer of a given size.
 * ------------------------------------------------------------------------- */
int voom_stream_read(const void* src, size_t n_bytes, uint32_t* sink, int workgroups,
                     hipStream_t stream);
/* The same for a row gather: reads row idx[i] (clamped into [0, n_base_rows))
 * of row_bytes (1 to 4 KiB, whole KiB) from base, and from base2 when it is
 * not NULL, for i < n_rows, four rows in flight per wavefront, 1 KiB per load
 * instruction.  bench.py times it over the position-free workload's page ids
 * in the K and V pools: the floor of reading those pages. */
int voom_gather_read(const void* base, const void* base2, size_t row_bytes, int n_base_rows,
                     const int32_t* idx, int n_rows, uint32_t* sink, int workgroups,
                     hipStream_t stream);
/* The data movement of the MLA latent kernel with no arithmetic: batch x
 * ranges x groups workgroups (the groups of a range on one XCD); each copies
 * its 64 query rows of q ([batch, 64 groups, 576] bf16, skipped when NULL)
 * and the 64-token tiles of its token range of pool ([num_slots, 64, 576]
 * bf16, page ids table[b][0..]) into LDS, two tile buffers, and writes
 * 64 x 512 fp16 of rows_out ([batch x ranges x groups, 64, 512]); sink has
 * one entry per workgroup.  bench.py times it at the latent kernel's own
 * decomposition (groups 2) and with one workgroup per range (groups 1): the
 * floors of the two ways of splitting the heads. */
int voom_tile_read(const void* pool, int num_slots, const int32_t* table, const void* q,
                   int batch, int max_pages, int ctx, int ranges, int groups, void* rows_out,
                   uint32_t* sink, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* VOOM_CALIBRATE_H */
