/*
 * CPU oracle for the OSSM scan kernels — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU kernels (loop order, parallel
 * decomposition and arithmetic of src/ossm/csrc/dlinoss_{imex1,imex2,im,ex}.cpp,
 * linoss_scan.cpp, selective_scan_cpu.cpp, sdlinoss_{imex1,imex2,im,ex}.cpp,
 * lru_scan.cpp / s5_scan.cpp, and the Python backwards of models/linoss.py:83-151
 * and models/lru.py:52-80 / s5.py:137-165).  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg load it, as the checker; the HIP library never
 * links or calls it.
 *
 * Built by oracle/Makefile with the reference's CPU flags (setup.py:47-55:
 * -O3 -ffast-math -fno-math-errno -fno-trapping-math -fopenmp).
 *
 * Pins: see tests/test_oracle.py — golden layer fixtures, the reference's own
 * CPU kernels compiled into oracle/_ref, closed forms and brute force.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

#define REAL float
#define SFX(x) x##_f32
#define EXP expf
#define FMA fmaf
#include "scan_oracle_body.h"
#undef REAL
#undef SFX
#undef EXP
#undef FMA

#define REAL double
#define SFX(x) x##_f64
#define EXP exp
#define FMA fma
#include "scan_oracle_body.h"
#undef REAL
#undef SFX
#undef EXP
#undef FMA

int oracle_num_threads(void) {
#ifdef _OPENMP
  extern int omp_get_max_threads(void);
  return omp_get_max_threads();
#else
  return 1;
#endif
}
