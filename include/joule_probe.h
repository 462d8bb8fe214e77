/*
 * joule_probe.h -- launch and hand-off cost probes (libjoule_probe.so).
 *
 * Measurement helpers with no counterpart in the reference: they time the
 * two ways a cross-block dependency can be crossed on the GPU, a kernel
 * boundary and an in-kernel "last block finishes" hand-off, so that the
 * figures the MoE block's launch structure rests on can be regenerated
 * (bench.py --probe).  Each call allocates, runs and frees its own buffers
 * and stream, and synchronises.  Return 0, or a negative code with
 * jmp_last_error() set.
 */
#ifndef JOULE_PROBE_H
#define JOULE_PROBE_H

#ifdef __cplusplus
extern "C" {
#endif

const char* jmp_last_error(void);

/* n dependent launches of a one-wave kernel on one stream (each reads the
 * word the previous one wrote), repeated reps times; use_graph = 1 captures
 * the n launches once into a HIP graph and replays it.  *us_per_launch =
 * elapsed / (n * reps). */
int jmp_launch_chain(int n, int use_graph, int reps, float* us_per_launch);

/* One launch of nblk blocks x 256 threads, each summing per_block floats
 * and storing its partial; handoff = 1 adds a release fence and a ticket
 * from one device-scope counter per block, and the last block sums the
 * partials.  *us_per_launch averages reps launches; *total (may be NULL)
 * receives the last-block sum (nblk * per_block with the hand-off on). */
int jmp_handoff(int nblk, int per_block, int handoff, int reps, float* us_per_launch, float* total);

/* A plain read stream: nbytes (a multiple of 4 * wave_bytes, at most
 * 4 GiB) read by waves of 64 lanes, each wave one contiguous piece of
 * wave_bytes (4096, 8192 or 16384) with every load in flight at once; reps
 * launches rotate over `regions` copies (at most 16, 6 GiB in all) so that
 * the bytes come from HBM.  *us_per_launch = elapsed / reps. */
int jmp_stream(unsigned long long nbytes, int wave_bytes, int regions, int reps, float* us_per_launch);

#ifdef __cplusplus
}
#endif

#endif
