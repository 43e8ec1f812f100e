/* hk phase stamps: a diagnostic entry point of lib/libhk_phases.so only.
 *
 * lib/libhk_phases.so is libhk.so built with -DHK_PHASE_STAMPS: the XCD-split
 * decode step then writes the 100 MHz real-time clock at fixed points of each
 * of its first 32 layers, per workgroup (16 slots: stagings, stores,
 * reductions) and per attention task (8 slots).  `bench.py --workload phases`
 * reads them to print the per-layer phase table.  No counterpart in the
 * reference, which has no such instrumentation; production callers load
 * libhk.so, which does not export this function. */
#ifndef HK_PHASES_H
#define HK_PHASES_H

#ifdef __cplusplus
extern "C" {
#endif

/* Copy the stamp tables to host memory: `phase` gets [256][32][16] and
 * `attn` [256][32][8] 64-bit clock values (either may be NULL), from the
 * last launch that wrote each one; with `clear` nonzero both tables are
 * zeroed afterwards, so the next copy shows only later launches.  Call it
 * with no launch in flight (it synchronises the device).  Returns 0 or an
 * HK_ERR_* code, the message in hk_last_error(). */
int hk_phase_stamps(void* phase, void* attn, int clear);

#ifdef __cplusplus
}
#endif

#endif /* HK_PHASES_H */
