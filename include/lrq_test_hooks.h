/*
 * lrq_test_hooks.h — test hooks exported by liblrq.so that are NOT part of the drop-in ABI.
 *
 * Nothing here stands in for a reference function; the declarations exist so that the test
 * suite can drive alternative kernels of an entry point and compare their results.  Callers
 * that replace the reference's operators use include/lrq.h only.
 */
#ifndef LRQ_TEST_HOOKS_H
#define LRQ_TEST_HOOKS_H

#include "lrq.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Same result as lrq_encode, always through the two-pass kernels (projection pass, then
 * residual/quantisation pass), so tests can compare the two paths on one shape. */
int lrq_encode_twopass(const lrq_tensors* t, const void* x, int64_t ldx, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LRQ_TEST_HOOKS_H */
