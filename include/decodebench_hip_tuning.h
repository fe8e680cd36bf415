/* decodebench_hip_tuning.h -- measurement hooks of libdecodebench_hip.so.
 *
 * Not part of the drop-in surface (include/decodebench_hip.h): these set the
 * launch geometry the library otherwise chooses itself, for the launch-shape
 * sweeps behind its defaults and for tests that force a code path.  No
 * counterpart in the reference.
 *
 * The knobs are per host thread: a value set on one thread changes only the
 * launches that thread makes, and a new thread starts from the defaults.
 * Knob values are read when a launch is made, so a captured hipGraph keeps
 * the values of its capture. */
#ifndef DECODEBENCH_HIP_TUNING_H
#define DECODEBENCH_HIP_TUNING_H

#ifdef __cplusplus
extern "C" {
#endif

/* Set a knob of the calling thread.  Keys and values:
 *  "gemv_waves_per_cu"   (<= 0: the default, 32)
 *  "gemv_mfma_min_batch" (0: automatic, 3 rows; 2 for the e4m3 norm and
 *                         gate/up modes and for plain rows longer than 4096)
 *  "f4_blocks_per_cu", "f4_min_tiles" (>= 1)
 *  "f4_waves"            (4 or 8 waves per workgroup, 0: automatic)
 *  "f4_merge"            (split merge: 0 automatic -- in the same launch where
 *                         the grid numbering puts each (batch, kv-head) pair
 *                         on one XCD of an 8-XCD device, else a second launch;
 *                         1 the same; 2 always a second launch)
 *  "f4_misplace"         (test hook, k >= 0: with the in-launch merge, split s
 *                         reports an XCD other than its own when
 *                         s % k == k - 1, so the merging workgroup of a pair
 *                         with such a split recomputes every split; 0 off)
 *  "f4_line"             (F4 score-operand layout: 0 automatic, 1 whole-line
 *                         K loads, 2 16 keys x 64 bytes per load)
 *  "f4_combine_groups"   (split groups of 32 threads per second-launch merge
 *                         workgroup: 1, 2, 4 or 8; 0 automatic)
 *  "f4_depth"            (tiles in flight per wave of the 8-wave whole-line F4
 *                         kernel: 1 or 2; 0 automatic)
 *  "gemv_long_kc"        (k-steps of 32 columns per chunk of the MFMA GEMVs
 *                         that stream their activations: 2 or 4; 0 automatic)
 *  "gemv_long_gpw"       (8-row groups per workgroup of the long-row kernel:
 *                         1, 2 or 4; 0 automatic)
 *  "gemv_long_stage"     (its activations: 1 loaded as B operands, 2 staged
 *                         through LDS; 0 automatic)
 *  "gemv_pair_min_batch" (batch rows from which the gate/up pair streams its
 *                         activations; 0 automatic, 17)
 *  "stream_waves"        (db_stream_read's waves per workgroup: 1, 2 or 4; 0
 *                         is 4)
 *  "gemv_pass_grid"      (one weight matrix above 16 batch rows on MFMA:
 *                         workgroups per 16-row pass, a multiple of 8; 0
 *                         automatic)
 *  "gemv_xb"             (1: 32-row passes with rows 16..31 of the
 *                         activations in LDS on the full grid; 0, the default,
 *                         off)
 *  "f4_launch"           (a call of F4 whose split merge runs in a second
 *                         launch makes only one of its two launches: 1 the
 *                         split kernel, 2 the merge, which then reads whatever
 *                         records the workspace holds; 0, the default, both.
 *                         For timing each half back to back; the output is not
 *                         the attention result)
 * Returns DB_OK, or DB_ERR_INVALID for an unknown key or a value outside the
 * key's range (nothing changes then). */
int db_tune(const char* key, int value);

/* How db_f4_splitkv would run a call of this shape on the current device
 * with the calling thread's knobs: *splits = the splits it uses (S capped at
 * the 16-row tiles of L), *launches = 1 (one split, or the split merge in the
 * same launch) or 2 (merge in a second launch).  DB_ERR_INVALID for a null
 * output or a shape db_f4_splitkv rejects; a HIP error code when the device
 * cannot be queried. */
int db_f4_launch_info(int B, int Hq, int Hkv, int L, int S, int* splits, int* launches);

/* The calling thread's current value of a knob (DB_ERR_INVALID for an
 * unknown key or a null argument). */
int db_tune_get(const char* key, int* value);

#ifdef __cplusplus
}
#endif

#endif /* DECODEBENCH_HIP_TUNING_H */
