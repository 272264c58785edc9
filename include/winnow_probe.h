/* Measurement probes for bench.py: libwinnow_probe.so, built beside libwinnow_hip.so.
 *
 * Not part of the drop-in and with no counterpart in the reference: nothing in
 * libwinnow_hip.so calls these, and a caller of the decode path has no reason to
 * load this library. Entry points return 0 on success and a negative status
 * otherwise, with the reason in wn_probe_last_error(). */
#ifndef WINNOW_PROBE_H
#define WINNOW_PROBE_H

#ifdef __cplusplus
extern "C" {
#endif

/* Thread-local message of this library's last failed call ("" after a success). */
const char* wn_probe_last_error(void);

/* The rate at which one CU's LDS serves the packed row scans' table lookups (8-byte
 * reads at random addresses of a pair table replicated once per lane of a half-wave,
 * as the 4-bit scans read theirs, every address moved to another row by one
 * instruction before its read as the scans form theirs; eight reads in flight per
 * wave) with waves_per_cu waves on every CU (1-16): *lookups_per_us_per_cu, timed
 * with HIP events over `iters` x 8 lookups per lane on the null stream. bench.py
 * turns it into the scans' LDS floor. */
int wn_probe_lds_lookup_rate(int waves_per_cu, int iters, double* lookups_per_us_per_cu);

#ifdef __cplusplus
}
#endif

#endif /* WINNOW_PROBE_H */
