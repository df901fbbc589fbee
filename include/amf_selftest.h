/* amf_selftest.h - libamf_selftest.so, device-side checks for the test suite.
 *
 * Test infrastructure with no counterpart in the reference and no place in
 * the drop-in ABI (amf_hip.h): it exposes the FP8 e4m3 encoder that the save
 * kernels inline, so the GPU tests can pin the gfx950 conversion instruction
 * against the portable encoder and an independent CPU encoder.
 */
#ifndef AMF_SELFTEST_H_
#define AMF_SELFTEST_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Mismatches reported in first_bad, three words each: the fp32 bits of the
 * first of four consecutive inputs (sign in bit 31), the portable encoder's
 * four codes, the kernels' four codes. */
#define AMF_SELFTEST_MAX_REPORT 8

/* Encodes every fp32 value with |x| <= 448 (both signs, 2 x 1,138,753,537
 * values) with the save kernels' encoder and with the portable bit-level
 * encoder, on the current device, and counts the four-value groups that
 * differ.  first_bad: host array of 3 * AMF_SELFTEST_MAX_REPORT words.
 * Synchronous; allocates and frees its own device memory.  Returns 0 or a
 * HIP error code (-1 for a null argument). */
int amf_selftest_e4m3_sweep(unsigned long long* mismatches, uint32_t* first_bad);

/* codes[i] = e4m3fn code of x[i] for i < n, with the save kernels' encoder
 * (inputs must already be clamped to [-448, 448], as the kernels do).  x and
 * codes are device pointers; asynchronous on `stream`.  Returns 0, a HIP
 * error code, or -1 for invalid arguments. */
int amf_selftest_e4m3_encode(const float* x, uint8_t* codes, int64_t n, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AMF_SELFTEST_H_ */
