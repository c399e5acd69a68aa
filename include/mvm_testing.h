/*
 * mvm_testing.h -- test hook of libmvm_scan.so.  Not part of the drop-in
 * boundary and with no counterpart in the reference; the GPU test suite uses
 * it to check the lane layout of the cross-lane reductions on the device.
 */
#ifndef MVM_TESTING_H
#define MVM_TESTING_H

#ifdef __cplusplus
extern "C" {
#endif

/* One wave: lane l holds x_j = 1000*j + l (j = 0..3).  Writes 128 floats to
 * device memory `out`: [0,64) the 4-lane state-group sum of x_0 per lane,
 * [64,128) the 16-channel reduction of (x_0..x_3) per lane. */
int mvm_selftest_lanes(float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MVM_TESTING_H */
