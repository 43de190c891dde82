/*
 * ref_det.c — the reference determinism gate (fp_determinism.c), compiled
 * from /root/reference without its main, exporting fp_det_compute().
 * TEST INFRASTRUCTURE ONLY (built into oracle/_ref/).
 */
#define FP_DET_NO_MAIN
#include "fp_determinism.c"
