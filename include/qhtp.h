/*
 * qhtp.h -- C ABI of libqhtp, the MI355X (gfx950) implementation of qcom_htp's two hot
 * paths: the QNN-semantics quantized matmul family and the GDN/KDA triangular solve.
 *
 * Conventions
 *   - Plain pointers and sizes only.  Every pointer named *_dev is device memory on the
 *     current HIP device; everything else is host memory.
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream).  Run entry
 *     points are stream-ordered and never synchronise the host.
 *   - Run entry points allocate nothing.  qh_qmm_prepare allocates the prepared weight
 *     state (device memory) once; qh_qmm_release frees it.
 *   - Every entry point validates its arguments and returns a status; no entry point
 *     returns QH_STATUS_OK for a shape it did not compute.  qh_last_error() gives a
 *     human-readable reason for the last failure on the calling thread.
 *   - Prepared handles are read-only during runs, so concurrent runs on different streams
 *     or host threads are safe, with one exception: qh_qmm_run_chain_noalloc keeps its
 *     intermediate results in one static array per device, so its calls that overlap on
 *     one device race and must be serialised by the caller.  Besides that array, the
 *     library holds only the per-thread error text and per-device caches of device
 *     attributes (atomic, set once per device).
 */
#ifndef QHTP_H_
#define QHTP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  Values 0..3 mirror HmStatus of the reference's prepared-run ABI
 * (example/handwritten_hmx_matmul/include/handwritten_hmx_matmul.h:11-16). */
typedef enum qh_status {
  QH_STATUS_OK = 0,
  QH_STATUS_INVALID_ARGUMENT = 1,
  QH_STATUS_UNSUPPORTED = 2,
  QH_STATUS_RUNTIME_ERROR = 3,
  QH_STATUS_SHAPE_UNSUPPORTED = 4,
} qh_status;

/* Replaces hm_status_string (handwritten_hmx_matmul.h:52). */
const char *qh_status_string(qh_status status);

/* Text of the last error raised on the calling thread ("" if none). */
const char *qh_last_error(void);

/* Library version as 0xMMmmpp. */
uint32_t qh_version(void);

/* ------------------------------------------------------------------------------------ */
/* Quantized matmul family                                                               */
/* ------------------------------------------------------------------------------------ */

/* Weight storage handed to qh_qmm_prepare (host memory, logical [N][K] order). */
typedef enum qh_weight_format {
  QH_WEIGHT_I8 = 0,      /* int8 codes in [-127, 127], per-output-channel scale            */
  QH_WEIGHT_I4 = 1,      /* int4 codes in [-7, 7] (one per int8), per-output-channel scale */
  QH_WEIGHT_I4_LPBQ = 2, /* int4 codes in [-7, 7] times a per-(channel, K-block) integer  */
                         /* scale in [1, 16], under a per-output-channel scale             */
  QH_WEIGHT_I4_GROUP = 3, /* int4 codes in [-7, 7] (int8 storage, [-127, 127] accepted) with */
                          /* one float32 scale per (channel, group_size-deep K group) and a  */
                          /* float bias: the per-group schema of                             */
                          /* generate_qnn_matmul_python_cases.py:392-423,460-470             */
  QH_WEIGHT_I16 = 4,     /* int16 codes [N][K] (weight16_nk): the W16A16 weight, computed as */
                         /* two int8 byte planes (docs/w16a16_is_two_w8a16.md:13-45); only   */
                         /* qh_qmm_accumulate and qh_qmm_run_contract apply to it            */
} qh_weight_format;

/*
 * One quantized matmul  out[M,N] = requant( (act[M,K] - act_zp) @ W[N,K]^T + bias[N] ).
 *
 * Semantics are those of the reference's float-derived oracle
 * (scripts/generate_qnn_matmul_python_cases.py:446-481):
 *   x_deq = (act - act_zp) * act_scale                            (float64)
 *   w_deq = fl32(w_int * weight_scale[n])                        (float32 product)
 *   bias_deq = bias_q[n] * fl64(act_scale * weight_scale[n])
 *   out = clip(rint((x_deq @ w_deq^T + bias_deq) / out_scale + out_zp), 0, 2^out_bits - 1)
 * w_int is the int8/int4 code, or code * block scale for LPBQ.  Results are bit-exact
 * to that definition; the integer accumulation is exact.
 *
 * Shapes: K % 32 == 0, N % 32 == 0, K <= 65536, N <= 2^20; M is given per run (any M >= 1).
 * act_bits / out_bits: 8 (uint8) or 16 (uint16).  LPBQ blocks: 32 or 64 along K.
 *
 * Replaces the reference op-package kernels HmxU8I8ToU8MatMul / HmxU8I4ToU8MatMul /
 * HmxU16I8ToU16MatMul / HmxU16I4ToU16MatMul and the LPBQ expand pre-op
 * HmxW4LpbqExpandToI8 (example/qnn_hmx_matmul_{u8i8,w4a8,w8a16,w4a16,common}/src; registration
 * at HmxU8I8ToU8MatMulOp.cpp:783-884), whose precompute step (:196-287) corresponds to
 * qh_qmm_prepare and whose hot callback (:289-405) corresponds to qh_qmm_run.
 */
typedef struct qh_qmm_desc {
  uint32_t k;
  uint32_t n;
  uint32_t act_bits;      /* 8 or 16 */
  uint32_t out_bits;      /* 8 or 16 */
  uint32_t weight_format; /* qh_weight_format */
  uint32_t lpbq_block;    /* 32 or 64 for QH_WEIGHT_I4_LPBQ, ignored otherwise */
  int32_t act_zp;         /* activation zero point, 0 <= act_zp < 2^act_bits */
  int32_t out_zp;         /* output zero point, 0 <= out_zp < 2^out_bits */
  double act_scale;       /* > 0 */
  double out_scale;       /* > 0 */
  const int8_t *weight_nk;         /* [N][K] int codes                                  */
  const uint8_t *lpbq_block_scale; /* [N][K / lpbq_block] in [1, 16] (LPBQ only)         */
  const float *weight_scale;       /* [N] per-output-channel scale, > 0                 */
  const int32_t *bias_q;           /* [N] int32 bias codes at act_scale*weight_scale, or NULL; */
                                   /* the integer contracts add it as it is              */
  /* Per-group and int16 weights (fields after bias_q are read only for these formats). */
  const float *group_scale;        /* [N][K / group_size] float32 scales (QH_WEIGHT_I4_GROUP) */
  uint32_t group_size;             /* K depth of a scale group: 64, 128, 256, ... (I4_GROUP)  */
  const float *bias_float;         /* [N] float bias added unquantised (I4_GROUP), or NULL   */
  const int16_t *weight16_nk;      /* [N][K] int16 codes (QH_WEIGHT_I16)                     */
} qh_qmm_desc;

typedef struct qh_qmm_prepared qh_qmm_prepared;

/* Build the device-resident prepared state (weight tiles, epilogue constants).
 * Synchronous; allocates device memory on the current device. */
qh_status qh_qmm_prepare(const qh_qmm_desc *desc, qh_qmm_prepared **out);

/* out_dev[M][N] (uint8 or uint16, row-major) from act_dev[M][K] (uint8 or uint16,
 * row-major; the reference's [1, M/32, 32, K] activation is this layout).  Picks the
 * MFMA GEMM for M > 16 and the streaming GEMV for M <= 16.  Per-group weights run on the
 * exact integer GEMM for every M; QH_WEIGHT_I16 returns QH_STATUS_UNSUPPORTED (use
 * qh_qmm_run_contract). */
qh_status qh_qmm_run(const qh_qmm_prepared *prep, uint32_t m, const void *act_dev, void *out_dev,
                     void *stream);

/* Same as qh_qmm_run with the kernel path forced: 0 = automatic, 1 = GEMM, 2 = GEMV. */
qh_status qh_qmm_run_path(const qh_qmm_prepared *prep, uint32_t m, const void *act_dev, void *out_dev,
                          uint32_t path, void *stream);

/* Exact int32/int64 accumulators acc[M][N] = sum_k (act - act_zp) * w_int, written as
 * int64 (the integer-accumulator contract of scripts/reconstruct_hmx_u8_drain.py:10-16).
 * w_int as for qh_qmm_run_contract (for QH_WEIGHT_I16: the int16 code, the identity
 * acc = 256 (act - zp) @ hi + (act - zp) @ lo of scripts/verify_w16a16_two_w8a16.py:21-57). */
qh_status qh_qmm_accumulate(const qh_qmm_prepared *prep, uint32_t m, const void *act_dev, int64_t *acc_dev,
                            void *stream);

/* The reference's integer output contracts, applied to the exact integer dot product
 * acc = sum_k (act - act_zp) * w_int of a prepared weight (w_int: the int8 / int4 code, code *
 * block scale for LPBQ, the raw code for per-group, the int16 code for QH_WEIGHT_I16);
 * qmax = 2^out_bits - 1, out_zp of the prepared descriptor, d = the divisor argument. */
typedef enum qh_contract {
  QH_CONTRACT_CLIP_I32 = 0,          /* clip(int32(acc + bias_q), 0, qmax), int32 arithmetic     */
                                     /* wrapping like numpy's: the "legacy" contract of          */
                                     /* gen_quant_chain.py:991-995 (_make_reference_step)        */
  QH_CONTRACT_CLIP_I64 = 1,          /* clip(acc + bias_q, 0, qmax) in int64: the unit-scale LPBQ */
                                     /* model hmx_w4a8_lpbq_scalar (HmxU8I4ToU8MatMulOp.cpp:210- */
                                     /* 233) with act_zp = 0 and bias_q = its "effective" bias   */
  QH_CONTRACT_DIV_RINT = 2,          /* clip(rint(double(acc) / d + out_zp), 0, qmax): the native */
                                     /* A16 contract (gen_quant_chain.py:986-987, d = 127 for W8; */
                                     /* d = 32767 is the W16A16 requantisation)                  */
  QH_CONTRACT_FLOOR256_DIV_RINT = 3, /* as DIV_RINT on floor(acc / 256) * 256: the native W4A16  */
                                     /* contract (gen_quant_chain.py:981-985, d = 7)             */
  QH_CONTRACT_ROUND_DIV = 4,         /* clip(round_half_away(acc / d) + out_zp, 0, qmax):        */
                                     /* hmx_w4a16_lpbq_scalar_native / round_div7               */
                                     /* (HmxU16I4ToU16MatMulOp.cpp:520-568, d = 7)               */
  QH_CONTRACT_U8_DRAIN = 5,          /* clip(trunc(double(acc + bias_q) * s / 512) + (b >> 7),   */
                                     /* 0, qmax): the closed-form A8 drain of                    */
                                     /* scripts/reconstruct_hmx_u8_drain.py:10-16,153-156, with  */
                                     /* act_zp = 128; `divisor` packs s as IEEE half bits (low   */
                                     /* 16) and the u16 baseline b (high 16).  A reconstruction  */
                                     /* of the hardware drain: no reference output pins it.      */
} qh_contract;

/* out_dev[M][N] (uint8 / uint16 per out_bits) = contract(acc) for act_dev[M][K]; exact int64
 * accumulation (i8 matrix cores), any M >= 1.  divisor >= 1 (ignored by the CLIP contracts;
 * the packed drain parameters for QH_CONTRACT_U8_DRAIN, whose half scale must be finite).
 * Replaces the reference's integer reference steps and scalar LPBQ fallbacks listed above. */
qh_status qh_qmm_run_contract(const qh_qmm_prepared *prep, uint32_t m, const void *act_dev, void *out_dev,
                              uint32_t contract, uint32_t divisor, void *stream);

/* `contract` value of qh_qmm_run_chain that selects the float-derived requantisation of
 * qh_qmm_run instead of an integer contract. */
#define QH_CONTRACT_NONE 0xFFFFFFFFu

/* A chain of `chain` identical matmuls, each one's output the next one's activation (the
 * reference's CHAIN graphs: gen_quant_chain.py:1346-1361, HmPreparedRun.chain of
 * handwritten_hmx_matmul.h:32; reference output = the step applied chain times, :1542-1544).
 * Needs K == N and act_bits == out_bits when chain > 1.  Each step is qh_qmm_run
 * (contract = QH_CONTRACT_NONE) or qh_qmm_run_contract(contract, divisor).  Intermediate results
 * alternate between out_dev and scratch_dev (the op's scratch operand: M x N output elements;
 * NULL allowed when chain == 1), so the last one lands in out_dev.  act_dev is only read.
 * An integer-contract chain with K == N <= 256 runs every step in one launch, with the
 * intermediate results on chip: scratch_dev is then required but left untouched. */
qh_status qh_qmm_run_chain(const qh_qmm_prepared *prep, uint32_t m, uint32_t chain, const void *act_dev,
                           void *out_dev, void *scratch_dev, uint32_t contract, uint32_t divisor, void *stream);

/* qh_qmm_run_chain that allocates nothing and takes no scratch operand.  No counterpart in the
 * reference; it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation).  The intermediate results
 * live in a static per-device array of 8 MiB: M x N output elements must fit in it (else
 * QH_STATUS_SHAPE_UNSUPPORTED).  All calls on one device share that array, so calls that overlap
 * on one device (other streams or threads) race; serialise them.  chain <= 1 uses no scratch. */
qh_status qh_qmm_run_chain_noalloc(const qh_qmm_prepared *prep, uint32_t m, uint32_t chain, const void *act_dev,
                                   void *out_dev, uint32_t contract, uint32_t divisor, void *stream);

typedef struct qh_qmm_info {
  uint32_t k, n, act_bits, out_bits, weight_format, lpbq_block;
  uint64_t device_bytes;      /* device memory held by the prepared state */
  uint64_t gemm_weight_bytes; /* bytes of the GEMM weight tiles */
  uint64_t gemv_weight_bytes; /* bytes the GEMV streams per call (weights + scales) */
} qh_qmm_info;

qh_status qh_qmm_query(const qh_qmm_prepared *prep, qh_qmm_info *info);

/* Frees the prepared state (synchronises the device first). NULL is accepted. */
qh_status qh_qmm_release(qh_qmm_prepared *prep);

/* Packed weight carriers of the reference: the byte streams its graph generator writes
 * (example/qnn_hmx_matmul_common/gen_quant_chain.py, pack orders of --w8-pack-order /
 * --w4-pack-order) and its op packages read.  K is the reduction depth, N the output channels;
 * "[R, C]" is the carrier tensor's trailing shape, stored row-major. */
typedef enum qh_weight_carrier {
  QH_CARRIER_I8_KN = 0,            /* [K, N] int8, logical order ("raw", gen_quant_chain.py:729-738)      */
  QH_CARRIER_W8_KMAJOR = 1,        /* [K, N] bytes: 32x32 K-major HMX tiles in (k tile, n tile) order,     */
                                   /* element (r, c) at (r/4)*128 + c*4 + r%4 (gen_quant_chain.py:285-303; */
                                   /* the output of HmxW4LpbqExpandToI8, HmxW4LpbqExpandToI8Op.cpp:84-101)  */
  QH_CARRIER_W8_KMAJOR_SPLIT128 = 2, /* one W8_KMAJOR stream per 128 channels (gen_quant_chain.py:306-314) */
  QH_CARRIER_W4_KMAJOR_N64 = 3,    /* [K, N/2]: 32x64 tiles of 1024 B, byte kg*128 + (n%32)*4 + kr holds   */
                                   /* channels n (low) and n+32 (high) of one k; the stream               */
                                   /* HmxU8I4ToU8MatMul reads (HmxU8I4ToU8MatMulOp.cpp:184-201)           */
  QH_CARRIER_W4_KPAIR = 4,         /* [K/2, N]: byte (k/2, n), even k low (HmxW4LpbqExpandToI8Op.cpp:35-41) */
  QH_CARRIER_W4_NMAJOR_KPAIR = 5,  /* the K-pair bytes in [N][K/2] memory order (gen_quant_chain.py:385-398) */
  QH_CARRIER_W4_NMAJOR_K4 = 6,     /* N32 tiles, then 8-k groups of k / k+4 pairs (gen_quant_chain.py:401-422) */
  QH_CARRIER_W4_KBLOCK32_NMAJOR_K4 = 7, /* 32-k blocks, then N32 tiles of k / k+4 pairs; the stream      */
                                   /* HmxU16I4ToU16MatMul reads (HmxU16I4ToU16MatMulOp.cpp:526-543)       */
  QH_CARRIER_W4_NPAIR_NMAJOR = 8,  /* [N/2, K]: channels n (even, low) and n+1 (gen_quant_chain.py:455-468) */
  QH_CARRIER_W4_NPAIR_TILE32_NMAJOR = 9, /* [N/2, K]: channels n and n+32 per 64 (gen_quant_chain.py:471-489) */
  QH_CARRIER_W4_FULL_CODES = 10,   /* [K, N]: one 4-bit code per byte (gen_quant_chain.py:619-627)          */
} qh_weight_carrier;

enum {
  QH_CARRIER_XOR80 = 1u,  /* every byte stored with its sign bit toggled (the DLC carrier form,  */
                          /* gen_quant_chain.py:645,676,716,738)                                  */
  QH_CARRIER_HILO = 2u,   /* W4: the first element of a pair in the high nibble ("_hilo" orders) */
  QH_CARRIER_BIASED = 4u, /* W4: nibble = code + 8 instead of two's complement                   */
};

/* Decodes a carrier into logical int8 codes weight_nk[N][K] (the layout qh_qmm_desc takes).
 * Host memory in and out; no device work.  packed_bytes must equal the carrier's size
 * (K*N for W8 carriers and W4_FULL_CODES, K*N/2 for the other W4 carriers).  Shape rules of
 * the generator apply (K, N multiples of 32; N multiple of 64 / 128 where the layout tiles N
 * by 64 / 128).  Replaces the per-element readers of the op packages
 * (HmxU8I4ToU8MatMulOp.cpp:178-201, HmxU16I4ToU16MatMulOp.cpp:514-543) and the prepare-time
 * unpacking they imply. */
qh_status qh_weight_unpack(uint32_t carrier, uint32_t flags, const uint8_t *packed, size_t packed_bytes, uint32_t k,
                           uint32_t n, int8_t *weight_nk);

/* The HmxW4LpbqExpandToI8 op on device memory (HmxW4LpbqExpandToI8Op.cpp:47-104):
 * weight_lpbq_dev [K/2, N] K-pair int4 bytes (QH_CARRIER_W4_KPAIR), block_scale_dev
 * [N * K/32] uint8 integer scales (index n * K/32 + k/32) ->
 * expanded_dev [K, N] bytes = sat_i8(q4 * scale) in the QH_CARRIER_W8_KMAJOR stream.
 * K % 32 == 0, N % 32 == 0.  Stream-ordered, allocates nothing. */
qh_status qh_w4_lpbq_expand_to_i8(const uint8_t *weight_lpbq_dev, const uint8_t *block_scale_dev,
                                  uint8_t *expanded_dev, uint32_t k, uint32_t n, void *stream);

/* ------------------------------------------------------------------------------------ */
/* GDN / KDA triangular solve  T = (I - A)^-1, A strictly lower triangular per head      */
/* ------------------------------------------------------------------------------------ */

typedef enum qh_gdn_precision {
  QH_GDN_FP32 = 0,     /* fp32 diagonal solves; merges on bf16 hi/lo split MFMA products with
                          fp32 accumulation (rel. Frobenius <= 1e-4)                           */
  QH_GDN_BF16 = 1,     /* fp32 diagonal solves, bf16 MFMA merges with fp32 accumulation        */
  QH_GDN_OP_MODEL = 2, /* qh_gdn_solve_u16 only, C <= 64: the GdnSolve op's own scalar model,
                          code for code (gdn_solve_core.h:28-83): int16 diagonal solves at the
                          internal scale 2/32767, float32 merges, lroundf requant             */
} qh_gdn_precision;

/* A_dev: float32 [heads][C][C] row-major, only the strictly lower triangle is read.
 * T_dev: float32 [heads][C][C]; the full matrix is written (zeros above the diagonal).
 * C % 16 == 0, 16 <= C <= 256.  Replaces the fp64 recurrence of
 * scripts/gdn_ref_kernel.py:84-87 and the block solve of
 * example/gdn_native/solve_op/src/gdn_solve_core.h:28-83. */
qh_status qh_gdn_solve_f32(const float *A_dev, float *T_dev, uint32_t heads, uint32_t C, uint32_t precision,
                           void *stream);

/* Quantized I/O contract of the reference's GdnSolve op and bare-metal gdnbm_solve
 * (example/gdn_native/solve_op/src/GdnSolveOp.cpp:185-254; baremetal/inc/gdnbm.idl:7-13):
 * A_dev uint16 codes [heads][C][C], A = (code - zpA) * sA; T_dev uint16 codes
 * T_code = clip(rint(T / sT) + zpT, 0, 65535), zeros (= zpT) above the diagonal.
 * With QH_GDN_OP_MODEL (C <= 64): the op's codes exactly, A_int16 = (int16)(code - zpA) and
 * T_code = (uint16)(clip(lroundf(T / sT), +-32767) + zpT) (GdnSolveOp.cpp:201-208). */
qh_status qh_gdn_solve_u16(const uint16_t *A_dev, uint16_t *T_dev, uint32_t heads, uint32_t C, int32_t zpA,
                           int32_t zpT, float sA, float sT, uint32_t precision, void *stream);


/* Fused GDN chunk products (the intra-chunk half of the gated delta rule,
 * scripts/gdn_ref_kernel.py:71-89).  For every batch b, chunk c of `chunk` tokens and head h:
 *   K^ = l2norm(K) (eps 1e-6), g = cumsum of the per-token log decay gc inside the chunk,
 *   A_ij = -beta_i (K^_i . K^_j) e^{g_i - g_j} for i > j,  T = (I - A)^-1,
 *   U = T (beta * V),  W = T (beta * K^)   [W = T (beta * K^ * e^g) with QH_GDN_W_DECAY].
 * k_dev, v_dev: bf16 bit patterns [batch][tokens][heads][head_dim]; g_dev (gc) and beta_dev:
 * float32 [batch][tokens][heads]; w_dev, u_dev: [batch][tokens][heads][head_dim], bf16 bit
 * patterns, or float32 with QH_GDN_OUT_F32.  head_dim == 128, chunk in {64, 128, 256},
 * tokens % chunk == 0.  bf16 MFMA with fp32 accumulation (tolerance: the bf16 bound, 1.05e-2
 * relative Frobenius against float64).  Buffers must be 16-byte aligned. */
enum {
  QH_GDN_W_DECAY = 1u, /* W = T (beta * K^ * e^g) (the reference kernel's form)           */
  QH_GDN_OUT_F32 = 2u, /* W and U (qh_gdn_chunk_state: o) as float32 instead of bf16      */
  QH_GDN_WU_F32 = 4u,  /* qh_gdn_chunk_state: w_dev and u_dev hold float32, not bf16      */
};
qh_status qh_gdn_chunk_uw(const uint16_t *k_dev, const uint16_t *v_dev, const float *g_dev, const float *beta_dev,
                          void *w_dev, void *u_dev, uint32_t batch, uint32_t tokens, uint32_t heads,
                          uint32_t head_dim, uint32_t chunk, uint32_t flags, void *stream);

/* qh_gdn_chunk_uw with a cap on the persistent grid: at most max_workgroups workgroups walk the
 * (batch, chunk, head) items (0 = as many as are resident on the device at once).  A cap leaves
 * compute units to concurrent work on other streams; results do not depend on it.  No
 * counterpart in the reference (its chunk loop is the sequential Python of
 * scripts/gdn_ref_kernel.py:91-101). */
qh_status qh_gdn_chunk_uw_ex(const uint16_t *k_dev, const uint16_t *v_dev, const float *g_dev, const float *beta_dev,
                             void *w_dev, void *u_dev, uint32_t batch, uint32_t tokens, uint32_t heads,
                             uint32_t head_dim, uint32_t chunk, uint32_t flags, uint32_t max_workgroups,
                             void *stream);

/* GDN chunk recurrence (the inter-chunk half of the gated delta rule; replaces the stage-B lines
 * of gdn_chunk, scripts/gdn_ref_kernel.py:91-101, run over the chunk loop of gdn_kernel,
 * :104-131).  For every batch b and head h, over the chunks of 64 tokens in order, with the
 * state S (128 x 128, keys x values) carried from s_in_dev (NULL: zero) to s_out_dev:
 *   q^ = l2norm(q) / sqrt(128), k^ = l2norm(k), g = cumsum of gc inside the chunk,
 *   P = (q^ k^T) e^{g_i - g_j} (j <= i), v_new = U - W S, o = (q^ e^g) S + P v_new,
 *   S = S e^{g_last} + (k^ e^{g_last - g})^T v_new,
 * where W, U are qh_gdn_chunk_uw's outputs for chunk 64 with QH_GDN_W_DECAY.
 * q_dev, k_dev: bf16 bit patterns [batch][tokens][heads][128]; g_dev (gc): float32
 * [batch][tokens][heads]; w_dev, u_dev: [batch][tokens][heads][128] bf16 bit patterns, or float32
 * with QH_GDN_WU_F32; o_dev: the same layout, bf16, or float32 with QH_GDN_OUT_F32;
 * s_in_dev, s_out_dev: float32 [batch][heads][128][128] (s_out_dev must not alias s_in_dev).
 * head_dim == 128, chunk == 64, tokens % 64 == 0 (zero-pad: zero q, k, v, beta and gc tokens
 * leave o and S unchanged).  precision: QH_GDN_FP32 (bf16 hi/lo split products, fp32
 * accumulation) or QH_GDN_BF16.  Buffers must be 16-byte aligned. */
qh_status qh_gdn_chunk_state(const uint16_t *q_dev, const uint16_t *k_dev, const float *g_dev, const void *w_dev,
                             const void *u_dev, const float *s_in_dev, float *s_out_dev, void *o_dev, uint32_t batch,
                             uint32_t tokens, uint32_t heads, uint32_t head_dim, uint32_t chunk, uint32_t flags,
                             uint32_t precision, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* QHTP_H_ */
