/* fcmoe_probe.h -- measurement probes of libfcmoe_probe.so (bench only).
 *
 * Not part of the operator ABI (include/fcmoe.h): these launches exist to
 * measure the chip (HBM streaming, the MFMA + LDS-read loop, MFMA beside
 * streaming waves, release fences, the prefill GEMM's load mix). Each returns
 * 0 or a negative FCMOE_E* code, with the message in fcmoe_last_error() of
 * libfcmoe.so. */
#ifndef FCMOE_PROBE_H_
#define FCMOE_PROBE_H_

#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Microbenchmarks behind the chip figures the design relies on (no
 * counterpart in the reference; bench.py --probe times them with events on
 * `stream`). Not part of the operator library: they are built into
 * libfcmoe_probe.so, which only the benchmark loads. Each enqueues one launch and returns at once. `sink` is a device
 * int32 buffer the kernels only write on an impossible condition.
 * _stream: `workgroups` x `waves` waves each stream src_bytes / (workgroups x
 *   waves) bytes (whole KiB, at least 8) of `src`: mode 0 nontemporal 16-byte
 *   loads to VGPRs (8-deep ring), mode 1 buffer_load ... lds into an 8 KiB
 *   per-wave LDS ring; lds_pad_bytes of dynamic LDS per workgroup (at least
 *   waves x 8 KiB in mode 1) limits the workgroups per CU.
 * _mfma: `workgroups` workgroups of `waves` waves, each looping `iters` times
 *   over (tile rows + channels) / 16 LDS fragment reads and the
 *   v_mfma_i32_16x16x64_i8 of one wave tile: tile 0 = 128x96 (waves 4 or 8),
 *   1 = 128x64 (8, 12), 2 = 96x80 (12), 3 = 64x96 (12), 4 = 64x64 (8, 16).
 * _mix: 256 workgroups (one per CU) of compute_waves MFMA + LDS-read waves
 *   (iters iterations of 2 reads and 7 MFMAs) and stream_waves waves that
 *   stream src_bytes / (256 x stream_waves) bytes each (accumulating with
 *   MFMAs when stream_mfma); compute_waves + stream_waves <= 16.
 * _fence: the mode-0 stream of _stream, then (release != 0) each wave stores
 *   1 KiB to `rows` ([workgroups x waves x 1 KiB]), issues an agent-scope
 *   release fence and the workgroup bumps counters[workgroup / 16] (zeroed
 *   by the caller); the 16th arrival of each group acquires and reads a
 *   neighbour's row.
 * _ring: the prefill GEMM's load mix without arithmetic: `workgroups`
 *   workgroups of 8 waves; per K chunk each wave loads 4 KiB of weights (a
 *   contiguous stream of src per workgroup) and a_loads KiB of A rows (8 rows
 *   x 128 bytes, 7168-byte stride, from a 2 MiB window of `arows` per XCD;
 *   arows >= 16 MiB) by buffer_load ... lds, keeping `lookahead` chunks in
 *   flight, with (barrier != 0) one workgroup barrier per chunk. Supported
 *   (lookahead, a_loads, barrier): (2,0,1), (2,2,1), (2,2,0), (4,2,1), (6,2,1).
 *   arows_bytes < 16 MiB is refused. The LDS ring has 2 stages whatever the
 *   lookahead (6 stages of this mix would need 288 KiB): with lookahead 4 or
 *   6 chunks still in flight land on stages that later chunks also target.
 *   Nothing reads the ring, so this times the loads, not a usable ring.
 * _loop_dma: the prefill GEMM's K loop without HBM: 256 workgroups of 8
 *   waves, each wave a 128 x 64 tile (per iteration 6 LDS fragment reads
 *   ahead of the MFMAs, then one A read per row of 4 MFMAs, as the 256-row
 *   persistent tile). mode bit 0: one workgroup barrier per iteration; bit 1:
 *   each wave issues 4 buffer_load ... lds of 1 KiB per iteration (32 KiB per
 *   CU, from a 64 KiB window of src per XCD, i.e. L2 hits) into LDS the loop
 *   does not read; bit 2: before the barrier, wait for the previous
 *   iteration's loads. src_bytes >= 1 MiB. */
int fcmoe_probe_stream(const void* src, int64_t src_bytes, int workgroups, int waves, int mode, int lds_pad_bytes,
                       int* sink, hipStream_t stream);
int fcmoe_probe_mfma(int tile, int waves, int workgroups, int iters, int* sink, hipStream_t stream);
int fcmoe_probe_mix(const void* src, int64_t src_bytes, int compute_waves, int stream_waves, int iters,
                    int stream_mfma, int* sink, hipStream_t stream);
int fcmoe_probe_fence(const void* src, int64_t src_bytes, int workgroups, int waves, int release, int* counters,
                      void* rows, hipStream_t stream);
int fcmoe_probe_ring(const void* src, int64_t src_bytes, const void* arows, int64_t arows_bytes, int workgroups,
                     int lookahead, int a_loads, int barrier, int* sink, hipStream_t stream);
int fcmoe_probe_loop_dma(const void* src, int64_t src_bytes, int mode, int iters, int* sink, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FCMOE_PROBE_H_ */
