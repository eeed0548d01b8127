/*
 * VisionHOPE SRNL CPU oracle — TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library, and only as the checker (or as the timed CPU baseline).  The
 * product library (visionhope_amd/_lib/libvisionhope_hip.so) never links it
 * and has no CPU fallback.
 *
 * The reference implements SRNL only as CUDA source (no CPU path exists:
 * models/srnl.py:113-114, models/srnl_core/chunk.py:175-176), so this file is a
 * restatement of that CUDA arithmetic in plain C, in fp32 (same operation order
 * as the reference's per-thread loops) and in fp64.  Built with
 * -ffp-contract=off so that the fp32 variant is plain IEEE arithmetic.
 *
 * Pinned by tests/test_oracle_srnl.py against closed forms, invariants, an
 * independent NumPy fp64 formulation and planted mistakes (see srnl_line.inc).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    double step_scale;        /* VISIONHOPE_STEP_SCALE, chunk.py:44 */
    double min_retention;     /* VISIONHOPE_MIN_RETENTION, chunk.py:45 */
    double retention_bias;    /* VISIONHOPE_RETENTION_BIAS, chunk.py:46 */
    double injection_margin;  /* VISIONHOPE_INJECTION_MARGIN, chunk.py:47 */
    int spectral_clamp;       /* SPECTRAL_CLAMP, chunk.py:48 */
    double spectral_margin;   /* VISIONHOPE_SPECTRAL_MARGIN, chunk.py:49 */
} oracle_consts;

#define REAL float
#define FN(name) name##_f32
#define SQRT sqrtf
#define LOG logf
#define EXP expf
#define EXPM1 expm1f
#define NEXTAFTER nextafterf
#include "srnl_line.inc"
#undef REAL
#undef FN
#undef SQRT
#undef LOG
#undef EXP
#undef EXPM1
#undef NEXTAFTER

#define REAL double
#define FN(name) name##_f64
#define SQRT sqrt
#define LOG log
#define EXP exp
#define EXPM1 expm1
#define NEXTAFTER nextafter
#include "srnl_line.inc"

int oracle_abi_version(void) { return 1; }
