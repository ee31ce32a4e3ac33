/*
 * piper_probe.h -- C ABI of libpiper_probe.so, the measurement library beside the MI355X
 * (gfx950) Piper Attention backend.  Nothing here is part of the operator: bench.py and the
 * tests load this library to calibrate rooflines and to check the attention kernels'
 * probability-code packers.  No counterpart in the reference, whose benchmarks price kernels
 * against published peaks only.
 *
 * Status codes: 0 on success, otherwise 1 (invalid argument), 2 (unsupported) or 3 (HIP error),
 * with a thread-local description from piper_probe_last_error().
 */
#ifndef PIPER_PROBE_H
#define PIPER_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PIPER_PROBE_ABI_VERSION 3

int piper_probe_abi_version(void);
const char* piper_probe_last_error(void);

/* ---------------------------------------------------------------------------------------
 * Dense MFMA rate.  Runs `workgroups` x 512 threads on `stream`; each wave issues
 * 4 * `iterations` MFMAs on four accumulator chains with all-ones operands (INT8 1, FP8 E4M3
 * 1.0), so that events around the launch give the sustained matrix-core rate at the running
 * clock: 4 * iterations * PIPER_MFMA_PROBE_OPS(kind) operations per wave.  `sink` receives one
 * 32-bit word per thread (workgroups * 512): the sum of the thread's 64 accumulators,
 * iterations * 2048 modulo 2^32 (INT8) or the FP32 bits of iterations * 4096 (FP8, exact for
 * iterations <= 4096), so a fast time cannot come from work the compiler removed.
 * ------------------------------------------------------------------------------------- */
#define PIPER_MFMA_PROBE_I8 0 /* v_mfma_i32_32x32x32_i8 */
#define PIPER_MFMA_PROBE_F8 1 /* v_mfma_f32_32x32x64_f8f6f4 on FP8 E4M3 */
/* Conversion checks of the attention kernels' probability codes (`iterations` is not used).  On
 * entry the 512 words of each workgroup's part of `sink` hold FP32 values; thread t packs values
 * 4 (t % 128) .. 4 (t % 128) + 3 with the kernels' own packer, the first value in byte 0, and
 * stores the word over word t.  P_CODES_U8: Piper Attention's UINT8 codes (round half to even,
 * saturated to [0, 255]; the reference rule is reference.py:104-107), each byte holding u - 128
 * as the PV MFMA's signed operand.  P_CODES_FP8: SageAttention2++'s FP8 E4M3 codes. */
#define PIPER_MFMA_PROBE_P_CODES_U8 2
#define PIPER_MFMA_PROBE_P_CODES_FP8 3
/* P_CODES_U8_SCALED: Piper Attention's scaled packer (the kernels' subtraction-free exp2 path):
 * thread t reads E = words 4 (t % 64) .. + 3 and the multiplier c = word 256 + 4 (t % 64) of its
 * workgroup's part and stores the UINT8 codes of the exact products E_i * c (round half to even;
 * defined for products in [0, 255.5)), as bytes u - 128 like P_CODES_U8. */
#define PIPER_MFMA_PROBE_P_CODES_U8_SCALED 4
#define PIPER_MFMA_PROBE_THREADS 512
#define PIPER_MFMA_PROBE_OPS(kind) ((kind) == PIPER_MFMA_PROBE_F8 ? 131072 : 65536)
int piper_mfma_probe(int32_t kind, int32_t workgroups, int32_t iterations, uint32_t* sink, void* stream);

/* ---------------------------------------------------------------------------------------
 * Issue probe: how MFMA execution, VALU issue and LDS reads of different waves share a SIMD.
 *
 * `workgroups` workgroups of 256 * waves_per_simd threads, each holding 100 KiB of LDS so that
 * a compute unit runs one of them (launch as many as the GPU has CUs).  Each wave learns its
 * slot on its SIMD (the order in which its workgroup's waves on that SIMD reach an LDS
 * counter), takes roles[slot], and runs that role's loop until s_memtime has advanced by
 * `cycle_budget` ticks, counting rounds; every wave of a workgroup starts after one barrier, so
 * the waves of a SIMD run their roles side by side.  Each role's loop body is fixed inline
 * assembly (the instruction stream does not depend on the compiler's scheduling):
 *
 *   IDLE        no work (the wave ends at once)
 *   MFMA        2 v_mfma_i32_32x32x32_i8 per round, two AGPR accumulator chains
 *   FMA         32 v_fma_f32 per round on 16 independent chains
 *   EXP         32 v_exp_f32 per round on 16 chains (x = 2^-x)
 *   CVT         32 v_cvt_pk_u8_f32 per round on 16 chains
 *   MIX         the attention loop's mix: per round 2 x (1 MFMA + 16 FMA + 4 cvt_pk_u8 + 2 exp)
 *   VALU_MIX    MIX without its MFMAs
 *   LDS         16 wave-wide ds_read_b128 (1 KiB each, distinct addresses) and a wait per round
 *   MFMA_FMA    2 x (1 MFMA + 16 FMA) per round in one wave
 *   MIX_VGPR    MIX with the MFMA accumulators in VGPRs instead of AGPRs (only beside MIX_VGPR or
 *               IDLE waves: it runs in a kernel of its own, status 2 otherwise)
 *   CLUSTER     8 MFMAs back to back (two AGPR chains), then 8 x (16 FMA + 4 cvt_pk_u8 + 2 exp):
 *               the attention loop's ratio with its MFMAs bunched as the score MFMAs are
 *   ADD_LIT     32 v_add_f32 per round with a 32-bit literal operand, 16 chains
 *   ADD_SGPR    32 v_add_f32 per round with an SGPR operand, 16 chains
 *   FMA_SPLIT   32 v_fma_f32 per round into 8 registers, the three sources in VGPR banks 0, 1, 2
 *               (bank = register number mod 4); fixed registers v64-v79, no dependences
 *   FMA_SAME    FMA_SPLIT with its first two sources in the same bank
 *   FMAC_SAME   32 v_fmac_f32 per round on 8 accumulators, each accumulator's bank that of the
 *               first source
 *   MAX3        32 v_max3_f32 per round, the sources in banks 0, 1, 2 (the attention loop's row max)
 *   PERM        32 v_perm_b32 per round, the sources in banks 0, 1, 2 (its code packing)
 *
 * A wave's record: its hardware ids, role, slot, the ticks its loop took and the rounds it
 * completed (rounds / ticks is its rate while the other waves of its SIMD ran theirs).
 * ------------------------------------------------------------------------------------- */
#define PIPER_ISSUE_IDLE 0
#define PIPER_ISSUE_MFMA 1
#define PIPER_ISSUE_FMA 2
#define PIPER_ISSUE_EXP 3
#define PIPER_ISSUE_CVT 4
#define PIPER_ISSUE_MIX 5
#define PIPER_ISSUE_VALU_MIX 6
#define PIPER_ISSUE_LDS 7
#define PIPER_ISSUE_MFMA_FMA 8
#define PIPER_ISSUE_MIX_VGPR 9
#define PIPER_ISSUE_CLUSTER 10
#define PIPER_ISSUE_ADD_LIT 11
#define PIPER_ISSUE_ADD_SGPR 12
#define PIPER_ISSUE_FMA_SPLIT 13
#define PIPER_ISSUE_FMA_SAME 14
#define PIPER_ISSUE_FMAC_SAME 15
#define PIPER_ISSUE_MAX3 16
#define PIPER_ISSUE_PERM 17
#define PIPER_ISSUE_ROLES 18
#define PIPER_ISSUE_MAX_WAVES_PER_SIMD 4
#define PIPER_ISSUE_RECORDS_PER_WORKGROUP 16

typedef struct piper_issue_record {
  uint32_t hw_id;  /* HW_REG_HW_ID: wave slot [3:0], SIMD [5:4], CU [11:8], SH [12], SE [15:13] */
  uint32_t xcc_id; /* HW_REG_XCC_ID */
  uint32_t role;
  uint32_t slot;   /* the wave's slot on its SIMD within its workgroup */
  uint64_t cycles; /* s_memtime ticks of the wave's loop */
  uint32_t rounds; /* loop rounds completed */
  uint32_t check;  /* depends on every result of the loop (keeps the work live) */
} piper_issue_record;

typedef struct piper_issue_probe_args {
  int32_t waves_per_simd; /* 1 .. PIPER_ISSUE_MAX_WAVES_PER_SIMD */
  int32_t workgroups;     /* 1 .. 65536 */
  int32_t roles[PIPER_ISSUE_MAX_WAVES_PER_SIMD]; /* role of slot s; entries past waves_per_simd unused */
  int64_t cycle_budget;   /* 1000 .. 10^8 s_memtime ticks */
  piper_issue_record* records; /* workgroups * PIPER_ISSUE_RECORDS_PER_WORKGROUP; record w of workgroup g
                                  at g * 16 + w (waves w < 4 * waves_per_simd are written) */
} piper_issue_probe_args;

int piper_issue_probe(const piper_issue_probe_args* args, void* stream);

/* ---------------------------------------------------------------------------------------
 * Engine clock.  `workgroups` one-wave workgroups (1 .. 256; workgroup g runs on XCC g % XCCs)
 * each read the variable-frequency shader clock counter (s_memtime, HIP's clock64) and the
 * constant-rate wall clock counter (s_memrealtime, HIP's wall_clock64) when they start, sleep
 * until the wall clock has advanced by `duration_us` microseconds (1 .. 2 * 10^6; each wave also
 * stops after 2^20 sleeps), and read both again.  Record g = {wall0, clock0, wall1, clock1} at
 * records[4 g .. 4 g + 3]; *wall_clock_khz receives the wall counter's rate
 * (hipDeviceAttributeWallClockRate of the current device).  The engine clock over the wave's life
 * is (clock1 - clock0) / (wall1 - wall0) * wall_clock_khz kHz: launched on a second stream beside
 * a workload, it reads the clock the workload runs at (the waves use a few VGPRs and no LDS).
 * ------------------------------------------------------------------------------------- */
#define PIPER_CLOCK_PROBE_MAX_WORKGROUPS 256
int piper_clock_probe(int32_t workgroups, int64_t duration_us, uint64_t* records, int32_t* wall_clock_khz,
                      void* stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* PIPER_PROBE_H */
