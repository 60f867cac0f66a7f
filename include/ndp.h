/* ndp.h - C ABI of libndprobe: device ceilings of the GPU the benchmark runs
 * on, measured rather than taken from a data sheet.
 *
 * No counterpart in the reference (an ESP32 engine has no matrix cores). The
 * benchmark divides its prefill figure by the dense fp16 MFMA rate this
 * probe measures, beside the nominal 2.5 PFLOP/s, and reports the shader
 * clock the GPU holds under that load.
 *
 * Each kernel runs a register-only loop (no memory traffic inside it): every
 * wave reads the 64-bit shader cycle counter (s_memtime) and the constant-rate
 * real-time counter (s_memrealtime) before and after its loop, so the clock
 * is measured per wave, under the same load, without a profiler.
 */
#ifndef NDP_H
#define NDP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Loop bodies. */
#define NDP_MFMA_F16 0   /* nacc independent v_mfma_f32_32x32x16_f16 chains per wave, each MFMA
                            followed by nexp v_exp_f32 on independent registers (0..8) */
#define NDP_VALU_EXP 1   /* 8 independent chains of v_exp_f32 */
#define NDP_VALU_FMA 2   /* 8 independent chains of v_fma_f32 */

typedef struct {
    double ms;               /* kernel time between two HIP events */
    double clock_ghz;        /* mean over waves of cycles / real time */
    double cycles_per_iter;  /* mean shader cycles per loop iteration, per wave */
    double flops;            /* MFMA floating-point operations of the launch (MFMA kinds) */
    double valu_insts;       /* VALU instructions of the launch in the timed loops (wave-level) */
    uint32_t waves;          /* waves launched */
    uint32_t cus;            /* compute units of the device */
} ndp_result;

/* One launch of `kind` on the current device: blocks_per_cu * CUs work-groups
 * of 64 * waves_per_block threads, `iters` loop iterations per wave. nacc is
 * 1, 2 or 4 (MFMA kinds; ignored otherwise), nexp 0, 2, 4 or 8. Returns 0, or
 * -1 for bad arguments, -3 for a HIP error. */
int ndp_run(int kind, int nacc, int nexp, int blocks_per_cu, int waves_per_block, int iters, ndp_result *r);

#ifdef __cplusplus
}
#endif
#endif /* NDP_H */
