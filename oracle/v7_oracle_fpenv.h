/* v7_oracle_fpenv.h -- the reference's MXCSR mode around each oracle path function (TEST INFRASTRUCTURE).
 * See orc_set_reference_fp_env in v7_oracle.h. */
#ifndef V7_ORACLE_FPENV_H
#define V7_ORACLE_FPENV_H
#include <xmmintrin.h>

unsigned orc_fp_enter(void);
static inline void orc_fp_leave(const unsigned *old) { _mm_setcsr(*old); }
#define ORC_REFERENCE_FP_ENV \
    const unsigned orc_fp_saved_ __attribute__((cleanup(orc_fp_leave), unused)) = orc_fp_enter()

#endif
