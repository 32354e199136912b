/*
 * Rate probes for MI355X (gfx950) -- C ABI of libesa_probe.so.
 *
 * No counterpart in the reference: these measure, on the GPU they run on,
 * the rates the attention kernels are judged against -- dense bf16 MFMA
 * throughput, HBM read bandwidth, and the L2 -> LDS rate of the
 * buffer_load ... lds path the MFMA kernels stage K and V through.  They
 * are measurement tools (bench.py --peaks), not part of the attention path,
 * and live in their own library so libesa.so's interface stays the drop-in
 * one.
 *
 * Conventions are those of esa.h: an esa_status per call, arguments checked
 * on the host before any launch, device pointers owned by the caller,
 * asynchronous launches on `stream` (a hipStream_t as void*).  Each probe
 * writes one value per thread to `sink` (workgroups x 256 entries, capacity
 * `sink_elems`) so its work cannot be optimised away, and the value is a
 * closed form of the inputs the caller can check.
 */
#ifndef ESA_PROBE_H_
#define ESA_PROBE_H_

#include "esa.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Dense bf16 MFMA: each wave of `workgroups` 256-thread workgroups runs
 * `iters` rounds of four independent v_mfma_f32_32x32x16_bf16 chains on
 * operands held in registers (A and B all equal to `one`, a bf16 bit
 * pattern, so the compiler cannot fold them).  Work = workgroups * 4 waves
 * * iters * 4 * 32768 flop.  sink[t] = 64 * 16 * iters * one^2 (float), exact
 * for one = 1.0 and iters <= 16384.  workgroups in [1, 2^20], iters in
 * [1, 16384]. */
esa_status esa_probe_mfma_bf16(int32_t workgroups, int32_t iters, uint16_t one, float* sink,
                               int64_t sink_elems, void* stream);

/* Global memory -> LDS through buffer_load_dwordx4 ... lds, the MFMA
 * kernels' staging path: each workgroup copies `iters` 16 KB chunks of the
 * `region_bytes` region at src (chunk (workgroup * chunk_stride + i) mod
 * region_bytes / 16384) into two LDS buffers, two chunks in flight.  A
 * region of a few MB with a small chunk_stride stays resident in every
 * XCD's L2, so the rate is L2 -> CU; a region larger than the caches read
 * once (chunk_stride = iters) gives the HBM -> LDS rate.  Bytes moved =
 * workgroups * iters * 16384.  sink[t] = the sum of the eight 16-bit words
 * thread t's last DMA wrote to LDS (as uint32).  region_bytes a multiple of
 * 16384 in [16384, 2^31), src 16-byte aligned, workgroups in [1, 2^20],
 * iters in [1, 2^20], chunk_stride in [0, 2^20]. */
esa_status esa_probe_l2_to_lds(const void* src, int64_t region_bytes, int32_t workgroups,
                               int32_t iters, int32_t chunk_stride, uint32_t* sink,
                               int64_t sink_elems, void* stream);

/* HBM read: `workgroups` 256-thread workgroups stream `bytes` of src once
 * (16-byte loads, grid-stride, four in flight per thread) and sum the
 * 32-bit words each thread read, modulo 2^32, into sink[t].  bytes a
 * positive multiple of 64, src 16-byte aligned, workgroups in [1, 2^20]. */
esa_status esa_probe_hbm_read(const void* src, int64_t bytes, int32_t workgroups, uint32_t* sink,
                              int64_t sink_elems, void* stream);

/* Row gathers into LDS through buffer_load_dwordx4 ... lds, the band
 * kernels' access pattern: each workgroup copies `iters` rounds of 64 rows
 * of 256 bytes (16 lanes per row, four rows per DMA instruction, two rounds
 * in flight) into two LDS buffers; round i of workgroup b takes the 64 row
 * indices rows[((b * iters + i) * 64) mod n_rows ..] (int32, clamped to
 * [0, src_rows - 1]).  With src_rows * 256 bytes of a few MB the rows stay
 * in every XCD's L2, so the rate is L2 -> CU for scattered 256-byte rows.
 * Bytes moved = workgroups * iters * 16384.  sink[t] = the sum of the
 * eight 16-bit words thread t's last DMA wrote (as uint32).  src 16-byte
 * aligned, src_rows * 256 < 2^31, n_rows a positive multiple of 64, rows
 * 64-byte aligned, workgroups in [1, 2^20], iters in [1, 2^20]. */
esa_status esa_probe_gather_to_lds(const void* src, int64_t src_rows, const int32_t* rows,
                                   int64_t n_rows, int32_t workgroups, int32_t iters,
                                   uint32_t* sink, int64_t sink_elems, void* stream);

/* HBM gather: `workgroups` 256-thread workgroups read the n_rows rows
 * rows[0 .. n_rows) (int32 indices, device memory) of 256 bytes each from
 * src -- the access pattern of the decode step's K / V row gathers -- 16
 * lanes per row, eight rows per lane in flight, and sum the 32-bit words
 * each thread read, modulo 2^32, into sink[t].  Indices are clamped to
 * [0, src_rows - 1] on the device.  src 16-byte aligned, src_rows >= 1,
 * n_rows >= 1, workgroups in [1, 2^20]. */
esa_status esa_probe_gather_read(const void* src, int64_t src_rows, const int32_t* rows,
                                 int64_t n_rows, int32_t workgroups, uint32_t* sink,
                                 int64_t sink_elems, void* stream);

/* LDS operand reads of the band forward at head_dim 128: each wave of
 * `workgroups` 256-thread workgroups reads its own 16-row slot (16 x 256
 * bytes of 16-bit ones) `iters` rounds in one pattern: 0 = the K operand's
 * ds_read_b128 with the kernels' swizzle, 1 = the V^T operand's
 * ds_read_b64_tr_b16 with the kernels' swizzle, 2 = ds_read_b64_tr_b16 over
 * contiguous 16-dim slices with a swizzle that gives each 16-lane group
 * eight distinct 16-byte bank groups, 3 = pattern 0 unswizzled.  LDS
 * instructions per wave: 4 iters (patterns 0, 3) or 8 iters (1, 2).
 * sink[t] = 32 * iters (the sum of the 16-bit words thread t read).
 * pattern in [0, 3], workgroups and iters in [1, 2^20]. */
esa_status esa_probe_lds_read(int32_t pattern, int32_t workgroups, int32_t iters, uint32_t* sink,
                              int64_t sink_elems, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ESA_PROBE_H_ */
