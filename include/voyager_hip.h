/* voyager_hip.h -- C ABI of the MI355X (gfx950) quantized-operator library.
 *
 * The library executes the reference's `quantized_ops` operator path
 * (src/voyager_compiler/ops/quantized.py, ops/layout.py) on the GPU.  The
 * Python package `voyager_amd` registers torch.library kernels under the same
 * operator names and schemas and calls these entry points through ctypes.
 *
 * Conventions
 *  - Every entry point returns 0 (VH_OK) or a nonzero status; the message of
 *    the last failure on the calling thread is returned by vh_last_error().
 *  - Pointers are device pointers; sizes are element counts; every launch is
 *    asynchronous on the caller's stream and the library never allocates,
 *    frees or synchronises (safe under stream capture).
 *  - "Reference form" (ref-form) outputs are what the reference schema
 *    returns: codes and scales as floating tensors of the input's dtype.
 *    "Packed" outputs hold one byte per code (and per block scale).
 */
#ifndef VOYAGER_HIP_H
#define VOYAGER_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* vh_stream_t; /* == hipStream_t */

/* status */
#define VH_OK 0
#define VH_EINVAL 1
#define VH_ELAUNCH 2

/* element dtypes of tensors crossing the boundary */
#define VH_BF16 0
#define VH_F32 1
#define VH_F16 2
#define VH_U8 3
#define VH_I64 4

/* format kinds (what a 65,536-entry quantization map computes) */
#define VH_FMT_IDENTITY 0 /* entry i == pattern i (get_quantization_map(None)) */
#define VH_FMT_INT 1      /* clamp(round(v), p0, p1) */
#define VH_FMT_MINIFLOAT 2 /* p0 exponent bits, p1 mantissa bits */
#define VH_FMT_POSIT 3    /* posit<p0, es=p1> */
#define VH_FMT_STEPS 4    /* non-decreasing step function, <= 64 levels */
#define VH_FMT_LUT 5      /* anything else: gathered from `lut` */

#define VH_FMT_SIGNED 1
#define VH_FMT_HW_E4M3 2 /* MINIFLOAT e4m3 (max 448) on the OCP fp8 converter */

#define VH_MAX_STEPS 64

/* A quantization map in closed form.  Filled by the host after verifying,
 * with vh_build_table, that the closed form reproduces the caller's table on
 * all 65,536 inputs. */
typedef struct vh_format {
  int32_t kind;
  int32_t p0, p1;   /* INT: lo, hi | MINIFLOAT: ebits, mbits | POSIT: nbits, es */
  int32_t flags;    /* VH_FMT_SIGNED */
  int32_t emin;     /* MINIFLOAT: smallest normal exponent, 2 - 2**(ebits-1) */
  float max_norm;   /* MINIFLOAT: largest finite magnitude */
  float clamp_bf16; /* MINIFLOAT: max_norm rounded to bfloat16 (the table's clamp) */
  float thresh;     /* POSIT: magnitudes below this flush to zero */
  int32_t nsteps;   /* STEPS: number of thresholds (levels - 1) */
  uint16_t nan_out; /* STEPS: bfloat16 bits of the entry every NaN input takes */
  uint16_t nan_level;
  uint16_t thr_key[VH_MAX_STEPS]; /* STEPS: order key of each level's first input */
  uint16_t val[VH_MAX_STEPS];     /* STEPS: bfloat16 bits of each level's entry */
  const void* lut;  /* LUT: 65,536 bfloat16 entries in device memory */
} vh_format;

/* Raised whenever an entry point's arguments or meaning change; a loader
 * compares vh_abi_version() with the VH_ABI_VERSION it was written against. */
#define VH_ABI_VERSION 2

const char* vh_last_error(void);
int vh_abi_version(void);

/* Rebuild a format's 65,536-entry table (bfloat16 bits, entry i for input
 * pattern i).  Replaces get_quantization_map's table construction
 * (quantization/fake_quantize.py:68-122) and verifies a classification. */
int vh_build_table(const vh_format* fmt, uint16_t* out, vh_stream_t stream);

/* Broadcast/block indexing of a per-element parameter (scale, zero point)
 * against a contiguous tensor of up to VH_MAX_DIMS dims: element (i_0..i_n)
 * reads param[sum_d (i_d / div[d]) * stride[d]].  div[d] is 1 or the block
 * size; stride[d] is 0 along broadcast dims.  This is repeat_per_block
 * (ops/quantized.py:124-144) and torch broadcasting in one rule. */
#define VH_MAX_DIMS 6
typedef struct vh_param {
  const void* ptr; /* NULL: absent */
  int32_t dtype;
  int32_t scalar;  /* 1: one value for every element */
  int64_t div[VH_MAX_DIMS];
  int64_t stride[VH_MAX_DIMS];
} vh_param;

/* quantize: out = F(round_c(round_c(x / scale) + zp)), F the map (or none),
 * round_c the rounding to the compute dtype.  Replaces
 * quantized_ops.quantize (ops/quantized.py:449-515) and, with no scale,
 * quantized_ops.vmap (ops/quantized.py:147-184).  out_dtype VH_U8 writes
 * packed codes. */
int vh_quantize(const void* x, int32_t x_dtype, const int64_t* shape, int32_t ndim,
                const vh_param* scale, const vh_param* zero_point, int32_t compute_dtype,
                const vh_format* fmt, void* out, int32_t out_dtype, vh_stream_t stream);

/* Measurement aid, no counterpart in the reference: the memory access of
 * vh_quantize's per-tensor bf16 -> one-byte path without its arithmetic --
 * reads nvec 16-byte groups of x, writes 8 bytes per group to out (each
 * group's high bytes) with the same workgroup shape, run length and cache
 * hints -- so a quantize's bandwidth can be read against what its access
 * pattern reaches on the part (bench.py reports both). */
int vh_stream_2to1(const void* x, int64_t nvec, void* out, vh_stream_t stream);

/* quantize with stochastic rounding (a `seed`): out = x / scale (+ zp) as
 * vh_quantize computes it, rounded to one of the two of `levels` around it
 * (levels ascending, device memory, bf16/fp16/fp32; a table's distinct
 * finite entries with one +0, or a codebook's entries).  Element i in the
 * row-major order of `shape` takes byte i % 4 of word (i % 16) / 4 of the
 * Philox4x32-10 draw of counter i / 16 keyed by *seed (int64, device
 * memory), and rounds away from zero when |v| + byte / 256 * (high - low)
 * >= |far| in float32.  Replaces _stochastic_round / _random_bytes /
 * _philox (ops/quantized.py:318-446) inside quantize (:449-515) and
 * quantize_mx (:1076-1115). */
#define VH_SR_MAX_LEVELS 16384
int vh_quantize_sr(const void* x, int32_t x_dtype, const int64_t* shape, int32_t ndim, const vh_param* scale,
                   const vh_param* zero_point, int32_t compute_dtype, const void* levels, int32_t levels_dtype,
                   int32_t nlevels, const int64_t* seed, void* out, int32_t out_dtype, vh_stream_t stream);

/* Codebook tables under a region grid (_region_view, ops/quantized.py:193-229):
 * `regions` tables; element (i_0..i_n) uses table
 * sum_d (i_d / region.div[d]) * region.stride[d] (region.ptr and dtype
 * unused; region.scalar = 1: one table).  edges: [regions][nedges] float32
 * in device memory, ascending, each the largest float32 not above the
 * caller's edge (a search of bfloat16 values against it answers as against
 * the edge itself).  entries: [regions][k] in device memory. */
typedef struct vh_codebook {
  const float* edges;
  int32_t nedges;
  int32_t k;
  const void* entries;   /* NULL (encode only): write the index */
  int32_t entries_dtype; /* VH_BF16, VH_F16 or VH_F32 */
  int64_t regions;
  vh_param region;
} vh_codebook;

/* quantize against a codebook: v = round_c(round_c(x / scale) + zp) as
 * vh_quantize computes it, then the count of the element's table's edges e
 * with !(e >= bf16(v)) (torch.searchsorted, left side: NaN past the end),
 * written as that index or as its entry (nedges == k - 1), in the compute
 * dtype.  Replaces encode (ops/quantized.py:232-287) as quantize
 * (:449-515) calls it for a codebook qmap, with its `output_code` bounds or
 * the midpoints of the entries. */
int vh_quantize_codebook(const void* x, int32_t x_dtype, const int64_t* shape, int32_t ndim,
                         const vh_param* scale, const vh_param* zero_point, int32_t compute_dtype,
                         const vh_codebook* cb, void* out, vh_stream_t stream);

/* Codebook lookup: out = round_out(round_x(entry[long(x)]) * scale) (no
 * scale: round_x(entry[long(x)])), the element's table's entry; negative
 * indices count from the end when wrap_negative (1-D indexing), NaN where
 * torch's indexing or gather would raise.  Replaces decode
 * (ops/quantized.py:290-315) and, with the block scale, _decode_and_scale
 * inside dequantize_mx (:574-591, 1118-1150). */
int vh_decode_codebook(const void* x, int32_t x_dtype, const int64_t* shape, int32_t ndim,
                       const vh_codebook* cb, int32_t wrap_negative, const vh_param* scale, void* out,
                       int32_t out_dtype, vh_stream_t stream);

/* max |x| (NaN propagating, zero past L) over blocks of `block` elements
 * along L of a contiguous [outer, L, inner] tensor: out [outer, ceil(L /
 * block), inner] in x_dtype.  One axis of the block reduction of
 * calculate_mx_qparam over several axes (ops/quantized.py:958-1031,
 * quantization/mx_utils.py:16-125); the axes are reduced one call at a time. */
int vh_block_amax(const void* x, int32_t x_dtype, int64_t outer, int64_t L, int64_t inner, int64_t block,
                  void* out, vh_stream_t stream);

/* dequantize: out = G((Fin(x) - zp) * scale).  Replaces
 * quantized_ops.dequantize (ops/quantized.py:518-571).  x_dtype VH_U8 reads
 * packed codes of fmt_in. */
int vh_dequantize(const void* x, int32_t x_dtype, const int64_t* shape, int32_t ndim,
                  const vh_param* scale, const vh_param* zero_point, int32_t compute_dtype,
                  const vh_format* fmt_in, const vh_format* fmt_out, void* out,
                  int32_t out_dtype, vh_stream_t stream);

/* Packed one-byte codes -> bfloat16 through a 256-entry bf16 table in device
 * memory: out[i] = lut[codes[i]], i < n.  The decode half of the posit8 GEMM
 * (`gemm.linear_posit8`: the lowered graph's direct cast of posit codes to
 * bf16, quantization/quantize_pt2e.py:557-561, before the bf16 GEMM).
 * codes and out 16-byte aligned. */
int vh_decode_bytes(const void* codes, int64_t n, const void* lut, void* out, vh_stream_t stream);

/* quantize_mx: block scales over `block` elements along the middle axis of a
 * contiguous [outer, L, inner] tensor, then codes.  Replaces
 * quantized_ops.quantize_mx (ops/quantized.py:1070-1115) and
 * calculate_mx_qparam (ops/quantized.py:958-1031; codes_out NULL).
 * pot != 0: scale = 2**(floor(log2 amax) - floor(log2 quant_max)); else
 * scale = scale_fmt(amax / quant_max [/ global_scale]).  Zero/NaN scales
 * become 1.  scale_dtype / codes_dtype VH_U8 write packed bytes (pot scales
 * as biased exponents: byte = e + pot_bias, 255 = inf); scale_dtype VH_F32
 * writes the scale values as float32.  code_lut (256 bytes, or NULL) remaps
 * packed codes, e.g. codebook indices to their int8 levels. */
int vh_quantize_mx(const void* x, int32_t x_dtype, int64_t outer, int64_t L, int64_t inner,
                   int64_t block, float quant_max, int32_t pot, const vh_format* scale_fmt,
                   const void* global_scale, int32_t gs_dtype, const vh_format* fmt,
                   void* scale_out, int32_t scale_dtype, int32_t pot_bias,
                   void* codes_out, int32_t codes_dtype, const uint8_t* code_lut, vh_stream_t stream);

/* vh_quantize_mx for the decode GEMV's activations (rows <= 16, blocks along
 * the last axis, a scale map, no power-of-two scales): the same scales and
 * codes, with the scales written as float32 block-major [L / block][16]
 * (row r of block b at b * 16 + r; rows past `rows` are not written) and the
 * codes as bytes through code_lut.  No counterpart in the reference (a
 * layout of quantized_ops.quantize_mx's outputs, ops/quantized.py:1070-1115,
 * for vh_gemv_nf4). */
int vh_quantize_mx_rows16(const void* x, int32_t x_dtype, int64_t rows, int64_t L, int64_t block,
                          float quant_max, const vh_format* scale_fmt, const vh_format* fmt, float* scale_out,
                          uint8_t* codes_out, const uint8_t* code_lut, vh_stream_t stream);

/* quantize_affine: per block min/max -> (scale, zero_point, codes).
 * Replaces quantized_ops.quantize_affine (ops/quantized.py:1218-1283).
 * codes_out NULL (fmt then optional): scale and zero point only. */
int vh_quantize_affine(const void* x, int32_t x_dtype, int64_t outer, int64_t L, int64_t inner,
                       int64_t block, float quant_min, float quant_max,
                       const vh_format* scale_fmt, const vh_format* fmt, void* scale_out,
                       void* zp_out, void* codes_out, int32_t codes_dtype, vh_stream_t stream);


/* ------------------------------------------------------------------ GEMM
 * C[M, N] = epilogue(A[M, K] . B[N, K]^T), operands K-contiguous ("xc,kc"),
 * fp32 accumulation on MFMA.  Replaces the GEMM inside quantized_ops.linear
 * / matmul (ops/layout.py:231-275) and the decode + GEMM of linear_mx /
 * matmul_mx (ops/quantized.py:651-805): decoded operands are formed in
 * registers while tiles are staged, never in HBM. */
#define OP_BF16 0 /* bfloat16 elements */
#define OP_FP8 1  /* OCP E4M3 bytes (fp8 MFMA); both operands or neither */
#define OP_MXI8 2 /* int8 codes * 2**(scale_byte - bias) per `block` elements */
#define OP_P8 3   /* posit8 codes, decoded through `lut` (256 bf16 entries) */

#define EPI_PLAIN 0       /* v = acc [* scale] [+ bias[n]] rounded to out_dtype */
#define EPI_ROUND_SCALE 1 /* v = bf16(bf16(acc) * scale): linear then dequantize */

typedef struct vh_epilogue {
  int32_t mode;
  int32_t out_dtype;    /* VH_BF16 or VH_F32 */
  const void* scale;    /* 0-d device scalar (alpha / dequantize scale) or NULL */
  int32_t scale_dtype;
  const void* bias;     /* [N] device vector or NULL */
  int32_t bias_dtype;
} vh_epilogue;

typedef struct vh_gemm_desc {
  const void* A;
  const void* B;
  void* C;
  int64_t M, N, K;
  int64_t lda, ldb; /* row pitch of A / B in bytes */
  int64_t ldc;      /* row pitch of C in elements */
  int32_t a_fmt, b_fmt;
  const void* a_scale; /* OP_MXI8: [M, a_scale_ld] bytes */
  const void* b_scale; /* OP_MXI8: [N, b_scale_ld] bytes */
  int64_t a_scale_ld, b_scale_ld;
  int32_t a_block, b_block;
  int32_t a_bias, b_bias;
  const void* lut;     /* OP_P8 decode table */
  int32_t tile_hint;   /* 0: automatic; 2: 256x128/4 waves, 3: 128x128/4, 4: 128x64/4,
                          5: 256x128/8 waves, 6: 256x256/8, 7: 128x256/8, 8: 128x128/8,
                          9: 256x128/8 (one-step prefetch), 10: 128x128/8 (one-step);
                          MX-int8 pairs: 50: 128x128/4 waves, 51: 128x128/8,
                          52: 128x64/4, 53: 256x128/8, 54: 64x128/4,
                          55: 128x128 and 56: 256x128 with 4 decoding +
                          4 multiplying waves */
  int64_t batch;       /* independent GEMMs (<= 1: one) */
  int64_t batch_stride_a, batch_stride_b; /* bytes (0: broadcast) */
  int64_t batch_stride_c;                 /* elements */
  int64_t batch_stride_a_scale, batch_stride_b_scale; /* bytes */
  vh_epilogue epi;
  /* Split of K across workgroups (MX-int8 pairs with batch <= 1, K % 64 ==
   * 0, N % 4 == 0 and blocks >= 16): each split leaves an fp32 partial in
   * `workspace` and a second kernel adds them in split order (deterministic)
   * and applies the epilogue.  split_k 0: automatic; the split needs
   * vh_gemm_workspace_bytes(desc) bytes of device memory at `workspace`
   * (16-byte aligned), else the GEMM runs unsplit. */
  int32_t split_k;
  void* workspace;
  int64_t workspace_bytes;
} vh_gemm_desc;

int vh_gemm(const vh_gemm_desc* desc, vh_stream_t stream);

/* Device bytes vh_gemm would use as split-K workspace for `desc` (0: none).
 * No counterpart in the reference, whose CPU GEMM needs no workspace. */
int64_t vh_gemm_workspace_bytes(const vh_gemm_desc* desc);

/* The kernel vh_gemm runs for `desc` (the same rule, evaluated on the host;
 * the output pointer C enters through its alignment): family 1 the
 * register-staged kernel (tiles 2..10 as tile_hint names them), 2 the
 * direct-to-LDS kernel on E4M3 operands (tiles 20..43), 3 the direct-to-LDS
 * kernel on bf16 operands (31, 33, 35, 37, 41), 4 the MX-int8 kernels
 * (50..56) with `splits` K splits.  No counterpart in the reference, whose
 * GEMM is one aten call; tests use it to assert which tile a shape takes. */
#define VH_GEMM_FAMILY_STAGED 1
#define VH_GEMM_FAMILY_DIRECT_FP8 2
#define VH_GEMM_FAMILY_DIRECT_BF16 3
#define VH_GEMM_FAMILY_MXI8 4
int vh_gemm_plan(const vh_gemm_desc* desc, int32_t* family, int32_t* tile, int32_t* splits);

/* ------------------------------------------------------------ MXNF4 GEMV
 * Decode-shape linear_mx (ops/quantized.py:651-723) for codebook weights
 * with 64-element blocks (lut4_to_int6 + fp8_e5m3 scales), M <= 16.
 *
 * vh_pack_nf4 bakes [N, K] level indices (0..15, one per byte) into the
 * GEMV's layout: for each 16-row x 64-column block, 64 lanes x 8 bytes, lane
 * l holding row l % 16, columns (l / 16) * 16 + [0, 16) as nibbles (column j
 * in the low nibble of byte j, column j + 8 in its high nibble).  Needs
 * N % 16 == 0 and K % 64 == 0.  Replaces the weight baking of
 * quantization/quantize_pt2e.py:819-828 for this format. */
/* MX-int8 linear at small M on exact fp16 operands.  vh_quantize_mx8_f16:
 * quantize_mx(x, int8, [-1], 16, 127, force_scale_power_of_two=True) of each
 * bf16 row of x [M, K] (ops/quantized.py:1070-1115), written decoded as
 * code * 2**(e - E_row) in fp16 (exact) with E_row, the row's largest finite
 * block exponent, in ex [M]; blocks more than 24 binades under E_row are
 * flushed to zero, blocks with a non-finite scale hold code * scale.
 * vh_mx8_bake_f16: packed weights (int8 codes [N, K], scale bytes
 * 2**(byte - scale_bias) per 16, 255 = inf) the same way, E per row in ew
 * [N] (weight baking, quantization/quantize_pt2e.py:819-828).
 * vh_gemm_mx8_f16: y = epilogue(sum_k x[m,k] w[n,k] * 2**(ex[m] + ew[n])),
 * the linear_mx GEMM (ops/quantized.py:651-723), as an fp16 GEMM over
 * `splits` K ranges into float32 partials `part` (splits * M * N floats)
 * and one reduction; with splits == 1 and a 16-byte aligned y (ldy and N
 * multiples of 8 for bf16, ldy of 4 for float32) the GEMM applies the
 * exponents and the epilogue itself and `part` may be null; tile 0:
 * 128x128, 1: 64x128, 2: 128x64, 3: 256x128, 4: 64x64 (two waves, eight
 * stages in flight: the small-M tile).  No
 * reference counterpart for the operand form: it is this library's
 * small-M layout of the same values. */
int vh_quantize_mx8_f16(const uint16_t* x, int64_t M, int64_t K, uint16_t* out, int32_t* ex, vh_stream_t stream);
int vh_mx8_bake_f16(const int8_t* codes, const uint8_t* scale, int32_t scale_bias, int64_t N, int64_t K,
                    uint16_t* out, int32_t* ew, vh_stream_t stream);
int vh_gemm_mx8_f16(const uint16_t* x, const int32_t* ex, const uint16_t* w, const int32_t* ew, int64_t M,
                    int64_t N, int64_t K, const vh_epilogue* epi, void* y, int64_t ldy, float* part,
                    int64_t part_bytes, int32_t splits, int32_t tile, vh_stream_t stream);

int vh_pack_nf4(const uint8_t* codes, int64_t N, int64_t K, uint8_t* out, vh_stream_t stream);

/* y[M, N] = sum over blocks b of s_x[m, b] * s_w[n, b] * sum_k Lx[m, k] Lw[n, k]
 * with Lx the activations' int8 levels [M, K], s_x float32 block-major
 * [K/64][16] (vh_quantize_mx_rows16), Lw = levels16[index] of the packed
 * weights (levels16: 16 int8 values in host memory, passed by value), s_w =
 * w_scale_fmt(byte) with the bytes tile-major [N/16][K/64][16] (column n of
 * block b at ((n / 16) * K/64 + b) * 16 + n % 16); int8 MFMA per block,
 * float32 accumulation, epilogue as vh_gemm (EPI_PLAIN). */
int vh_gemv_nf4(const int8_t* x_levels, const float* x_scale, int64_t M, const uint8_t* w_packed,
                const uint8_t* w_scale, const vh_format* w_scale_fmt, const int8_t* levels16, int64_t N,
                int64_t K, const vh_epilogue* epi, void* y, vh_stream_t stream);

/* vh_quantize_mx_rows16 + vh_gemv_nf4 for one bfloat16 row x[K], in one
 * launch: each 64-element block of x is quantized inside the GEMV
 * (quantize_mx(x, fmt, [-1], 64, quant_max, scale map x_scale_fmt),
 * ops/quantized.py:1070-1115, by the same block-scale and element-code
 * functions, so levels and scales are those of the two launches bit for
 * bit), its codes taken to levels through levels16.  Replaces, like
 * vh_gemv_nf4, quantized_ops.linear_mx at M = 1 (ops/quantized.py:651-723).
 * x_scale_fmt: a minifloat (not the E4M3 hardware form); x_fmt: an index
 * table (STEPS) of at most 16 levels. */
int vh_gemv_nf4_m1(const void* x, int32_t x_dtype, float quant_max, const vh_format* x_scale_fmt,
                   const vh_format* x_fmt, const uint8_t* w_packed, const uint8_t* w_scale,
                   const vh_format* w_scale_fmt, const int8_t* levels16, int64_t N, int64_t K,
                   const vh_epilogue* epi, void* y, vh_stream_t stream);

/* MXNF4 linear_mx at any M (prefill; ops/quantized.py:651-723 with the
 * operand decode of :574-591): x_idx [M, K] codebook indices (0..15, one
 * byte each, as quantize_mx packs them) with x_scale [M, K / 64] codes of
 * x_scale_fmt; the weight as vh_pack_nf4 bakes it (w_packed) with w_scale
 * tile-major [N / 16][K / 64][16] codes of w_scale_fmt (the decode GEMV's
 * operands).  y = epilogue(sum_k xd[m,k] wd[n,k]), xd = bf16(level[x_idx] *
 * x_scale) and wd likewise -- the reference's decoded operands exactly --
 * accumulated in float32.  Needs N % 16 == 0, K % 64 == 0.  tile 0 and
 * splits 0 choose (vh_gemm_nf4_plan); tile 1: 128 x 128, 2: 256 x 128;
 * with more than one K split the float32 partials go to `part` (splits * M
 * * N floats, ldy == N) and one reduction applies the epilogue. */
int vh_gemm_nf4(const uint8_t* x_idx, const uint8_t* x_scale, const vh_format* x_scale_fmt, int64_t M,
                const uint8_t* w_packed, const uint8_t* w_scale, const vh_format* w_scale_fmt,
                const int8_t* levels16, int64_t N, int64_t K, const vh_epilogue* epi, void* y, int64_t ldy,
                int32_t tile, int32_t splits, float* part, int64_t part_bytes, vh_stream_t stream);
/* The tile, split count and block rows vh_gemm_nf4 takes for a shape (the
 * caller's nonzero *tile / *splits are kept, the splits rounded to whole
 * ranges of 64-element blocks), so the caller can size its workspace. */
int vh_gemm_nf4_plan(int64_t M, int64_t N, int64_t K, int32_t* tile, int32_t* splits, int64_t* bm);
/* The operands of vh_gemm_nf4 decoded once to bfloat16, for the two-pass
 * prefill (decode, then the bf16 GEMM of vh_gemm): x_out [M, K] =
 * bf16(level[x_idx] * x_scale) and w_out [N, K] the weight's rows likewise,
 * bit for bit the operands vh_gemm_nf4 multiplies -- the reference's
 * decoded operands (_dequantize_mx, ops/quantized.py:574-591).  Either
 * output may be NULL to skip that operand.  Arguments as vh_gemm_nf4. */
int vh_nf4_decode_bf16(const uint8_t* x_idx, const uint8_t* x_scale, const vh_format* x_scale_fmt, int64_t M,
                       const uint8_t* w_packed, const uint8_t* w_scale, const vh_format* w_scale_fmt,
                       const int8_t* levels16, int64_t N, int64_t K, uint16_t* x_out, uint16_t* w_out,
                       vh_stream_t stream);

/* ------------------------------------------------- decoder-layer decode step
 * One decode step (a batch of single tokens, M <= 16) of a Llama-style layer
 * whose linears are MX-int8 (int8 codes, block 16 along K, power-of-two
 * scales: quantize_mx + linear_mx, ops/quantized.py:1122-1216 / :651-723)
 * and whose KV cache is KIVI: 2-bit group-wise affine codes
 * (quantize_affine / dequantize, ops/quantized.py:1218-1283 / :518-571; keys
 * grouped along tokens, values along channels, group 32) plus a
 * full-precision residual window (quant_folding.py:1025-1120).
 *
 * Each linear's input is handed over as its MX-int8 fake quantization
 * (code x 2**e, exact) in fp16, produced by the kernel that computes it.
 * Kernels report data they cannot represent by OR-ing VH_DECODE_ERR_* bits
 * into a caller-owned device int32 (`flag`); the caller checks it. */
#define VH_DECODE_ERR_FP16_RANGE 1   /* an activation block exceeds fp16 (|x| > 65504) */
#define VH_DECODE_ERR_WEIGHT_RANGE 2 /* a weight block exponent outside [-24, 5] */
#define VH_DECODE_ERR_KV_CODE 4      /* a folded KIVI chunk held a value whose code is NaN */
#define VH_DECODE_ERR_KV_FULL 8      /* the main cache had no room for a completed chunk */
#define VH_DECODE_ERR_KV_STATE 16    /* the cache state was out of range (nothing was computed) */
#define VH_KIVI_RES_CAP 128          /* residual window slots */

#define VH_GEMV_STORE 0    /* y = bf16(x W^T) */
#define VH_GEMV_RESIDUAL 1 /* y = bf16(bf16(x W^T) + residual) */
#define VH_GEMV_SWIGLU 2   /* y = bf16(silu(bf16(x Wg^T)) * bf16(x Wu^T)), fq_out = its fake quantization */

/* LlamaRMSNorm of each row of x [M, H] (bf16) with weight w [H]: h_out
 * (bf16, optional) and its MX-int8 fake quantization fq [M, H] (fp16 bits).
 * Replaces the rmsnorm + quantize_mx pair of a converted decoder layer. */
int vh_rmsnorm_mx8(const uint16_t* x, const uint16_t* w, int64_t M, int64_t H, float eps, uint16_t* h_out,
                   uint16_t* fq, int32_t* flag, vh_stream_t stream);

/* Bake MX-int8 weights [N, K] -- codes one int8 per byte and block scales as
 * biased exponent bytes 2**(byte - scale_bias), as vh_quantize_mx packs
 * them -- into the GEMV layout: w_codes N*K bytes, w_hb N*K/16 bytes.
 * paired != 0 interleaves rows [0, N/2) and [N/2, N) tile by tile (gate / up
 * projections for VH_GEMV_SWIGLU).  The operand holds a block's exponent
 * in the fp16 exponent field, so it must lie in [-24, 5]: with w_shift
 * (int32 [N], rows in the input order) each row whose nonzero blocks leave
 * that range is rebased to its largest exponent E (baked as e - (E - 5),
 * w_shift[n] = E - 5, the GEMV multiplying the row's sums back; blocks more
 * than 29 binades under E are flushed) and the others get 0; without it
 * such blocks set VH_DECODE_ERR_WEIGHT_RANGE.  An infinite block scale
 * always does.  Needs N % 16 == 0 (32 when paired) and K % 256 == 0.
 * Replaces the weight baking of quantization/quantize_pt2e.py:819-828 for
 * this format. */
int vh_mx8_bake(const uint8_t* codes, const uint8_t* scale, int32_t scale_bias, int64_t N, int64_t K,
                int32_t paired, uint8_t* w_codes, uint8_t* w_hb, int32_t* w_shift, int32_t* flag,
                vh_stream_t stream);

/* linear_mx of fake-quantized activations x_fq [M, K] (fp16 bits) and baked
 * MX-int8 weights with N output columns (2N baked rows for VH_GEMV_SWIGLU);
 * exact products, fp32 accumulation, bf16 output y [M, N] (optional for
 * SWIGLU), residual [M, N] for VH_GEMV_RESIDUAL, fq_out [M, N] (fp16 bits)
 * for SWIGLU.  tiles_per_block 1 or 2 (16 or 32 columns per workgroup,
 * STORE / RESIDUAL).  M <= 16, K % 256 == 0, N % 16 == 0.  Rebased
 * operands (optional, else null): row_exp [M] -- each row of x_fq holds
 * its values times 2**-row_exp[m] (vh_quantize_mx8_f16's exact fp16 rows),
 * w_shift -- the bake's row shifts; the sums are multiplied by
 * 2**(row_exp + w_shift) before the epilogue. */
int vh_gemv_mx8(const uint16_t* x_fq, int64_t M, int64_t K, const uint8_t* w_codes, const uint8_t* w_hb, int64_t N,
                int32_t mode, int32_t tiles_per_block, const uint16_t* residual, uint16_t* y, uint16_t* fq_out,
                const int32_t* row_exp, const int32_t* w_shift, int32_t* flag, vh_stream_t stream);

/* Bake a KIVI main cache: T tokens (T % 32 == 0, head_dim 128) of each of
 * P = batch x kv-heads sequences -- codes (0..3, one per byte) [P, T, 128]
 * and bf16 scale / zero point as quantize_affine returns them: keys
 * [P, T/32, 128] (grouped along tokens), values [P, T, 4] (grouped along
 * channels) -- into groups [g0, g0 + T/32) of a main cache with room for
 * group_cap groups of 32 tokens per sequence (main_out P * group_cap * 3072
 * bytes: per group key codes, value codes, key and value scale / zero point
 * as fp16 -- exactly the algorithmic 96 bytes per token per kv head).
 * Replaces the store of the main cache (quantize_affine,
 * codegen/transform/quant_folding.py:2213-2314). */
int vh_kivi_bake(const uint8_t* k_codes, const uint16_t* k_scale, const uint16_t* k_zp, const uint8_t* v_codes,
                 const uint16_t* v_scale, const uint16_t* v_zp, int64_t P, int64_t T, int64_t group_cap, int64_t g0,
                 uint8_t* main_out, vh_stream_t stream);

/* Fill the first n residual slots from k, v [P, n, 128] (bf16): kr and vr
 * are [P, 128 slots, 128] bf16. */
int vh_kivi_bake_residual(const uint16_t* k, const uint16_t* v, int64_t P, int64_t n, uint16_t* kr, uint16_t* vr,
                          vh_stream_t stream);

/* KIVI cache state, device int32[4]: {tokens in the main cache (a multiple
 * of 32), residual slots filled before the step (< 128), a counter the
 * advance kernel keeps at 0 between launches, unused}.  The step's position
 * is their sum.  The kernels read it on the device, so one captured step
 * replays at every position. */
typedef struct vh_kivi_desc {
  const uint16_t* qkv;     /* [batch, qkv_ld] bf16: nq query heads, nkv key heads, nkv value heads (pre-RoPE) */
  int64_t qkv_ld;
  const uint16_t* rope;    /* [2][max_pos][128] bf16: cos, then sin, of each position */
  int64_t max_pos;
  uint8_t* main;           /* main cache [P][group_cap][3072] (vh_kivi_bake) */
  int64_t group_cap;       /* groups of 32 tokens the main cache holds per sequence */
  uint16_t* kr;            /* residual window, bf16 [P][VH_KIVI_RES_CAP][128]: every slot is read (those past
                              the state's n_res are masked), this step's key and value land in slot n_res */
  uint16_t* vr;            /* the same for values */
  int32_t* state;          /* device int32[4], see above */
  int64_t batch, nkv, nq, head_dim; /* nq == 4 nkv, head_dim == 128 */
  float softmax_scale;     /* 1 / sqrt(head_dim) */
  float* part;             /* workspace of part_floats floats, 16-byte aligned */
  int64_t part_floats;     /* >= w(P, S, T) = r4(P (S + 1) 8) + r4(P S 512) + r4(P 4 T / 2), P = batch * nkv,
                              S = ceil(group_cap / 16), T = 32 group_cap + 128, r4 = round up to a multiple
                              of 4 */
  uint16_t* attn;          /* [batch, nq * 128] bf16 attention output (optional) */
  uint16_t* attn_fq;       /* [batch, nq * 128] fp16 bits: its MX-int8 fake quantization */
  int32_t* flag;
  int32_t advance;         /* nonzero: advance the state after the step (below) */
  vh_format scale_fmt;     /* advance: the scale / zero-point map of the fold (fp16_e5m10) */
  vh_format code_fmt;      /* advance: the code map of the fold (uint2) */
} vh_kivi_desc;

/* Decode attention over main + residual: RoPE on this step's query and key,
 * the key / value appended at residual slot n_res, then softmax(q K^T *
 * softmax_scale) V over the n_main + n_res + 1 positions (GQA, 4 query heads
 * per kv head), with the main keys dequantized and each score rounded as the
 * reference's bf16 eager attention rounds them.  Replaces the split-cache
 * attention of a converted decode graph (quant_folding.py:1025-1120 split,
 * :2391-2547 read path, eager attention).
 *
 * With desc->advance the step also does the cache bookkeeping: when it filled
 * the residual's last slot (n_res == 127), the 128 residual tokens are
 * quantized with the KIVI specs (quantize_affine through code_fmt /
 * scale_fmt, keys along tokens, values along channels, group 32) into the
 * next 4 groups of the main cache and the residual restarts; otherwise n_res
 * grows by one.  This replaces the fold of a completed chunk
 * (quant_folding.py:1994-2065, :2634-2700, move_folds_out) -- here on the
 * device, so replays need no host step.  A chunk with no room flags
 * VH_DECODE_ERR_KV_FULL and leaves the state; a value whose code is NaN
 * flags VH_DECODE_ERR_KV_CODE.  Without it the state is left as it was. */
int vh_kivi_attention(const vh_kivi_desc* desc, vh_stream_t stream);

/* ------------------------------------------------------- outliers (CSR)
 * The outlier path of an MX linear: activations whose magnitude reaches a
 * threshold are kept exact in a CSR stream of fixed capacity and multiplied
 * by the decoded weight beside the quantized GEMM.  CSR arrays: data
 * (values), indices (int32 columns), indptr (int32 row pointers, rows + 1
 * per matrix); capacity slots past the stored entries hold data 0 and index
 * -1.  A matrix holding more entries than its capacity keeps the first ones
 * in row-major order, and its row pointers are clamped at the capacity. */

/* filter_outlier (ops/quantized.py:1286-1374, _pad_csr :1292-1319) and the
 * filter of quantize_mx_outlier (:1396-1458): for each of `batch` dense row-major
 * [rows, cols] matrices of x (dtype VH_BF16 / VH_F16 / VH_F32), the
 * non-zero elements with |x| >= threshold (threshold already rounded to the
 * dtype, as torch compares a tensor with a Python float) form a CSR of
 * max_nnz slots per matrix (data in the input dtype, [batch, max_nnz];
 * indices [batch, max_nnz]; indptr [batch, rows + 1], plus indptr_offset);
 * inliers = x with every element whose magnitude reaches the threshold
 * zeroed.  Three launches: segment counts (and the inliers), a scan per
 * matrix, the fill.  work: vh_filter_outlier_workspace_bytes(batch, rows,
 * cols) bytes of device memory, 16-byte aligned (segment counts and the
 * outliers each segment keeps for the fill). */
int vh_filter_outlier(const void* x, int32_t dtype, int64_t batch, int64_t rows, int64_t cols, float threshold,
                      int64_t max_nnz, int32_t indptr_offset, void* data, int32_t* indices, int32_t* indptr,
                      void* inliers, void* work, int64_t work_bytes, vh_stream_t stream);

/* Workspace bytes vh_filter_outlier needs.  No counterpart in the
 * reference, whose CPU filter builds each matrix's CSR with
 * Tensor.to_sparse_csr. */
int64_t vh_filter_outlier_workspace_bytes(int64_t batch, int64_t rows, int64_t cols);

/* vh_filter_outlier with no workspace argument and no allocation, for
 * callers that cannot allocate device memory: code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc.  No counterpart in
 * the reference.  The workspace is the library's own fixed scratch of
 * VH_FILTER_NOALLOC_SCRATCH_BYTES per GPU (a device array each GPU the
 * library runs on holds until the process ends); sizes whose
 * vh_filter_outlier_workspace_bytes exceed it return VH_EINVAL with a
 * message.  Every call on one GPU shares that GPU's scratch: calls that
 * overlap on one GPU (different streams, threads) race. */
#define VH_FILTER_NOALLOC_SCRATCH_BYTES (8ll << 20)
int vh_filter_outlier_noalloc(const void* x, int32_t dtype, int64_t batch, int64_t rows, int64_t cols,
                              float threshold, int64_t max_nnz, int32_t indptr_offset, void* data, int32_t* indices,
                              int32_t* indptr, void* inliers, vh_stream_t stream);

/* slice_csr_tensor (ops/quantized.py:1493-1545) of one CSR matrix with
 * `rows` rows and `cap` slots (indptr[0] == 0), to out_cap slots.
 * dim 0: rows [start, end), pointers rebased to 0.  dim 1: columns
 * [start, end), entries compacted row by row in order and their columns
 * shifted by -start.  out_indptr has end - start + 1 (dim 0) or rows + 1
 * (dim 1) entries. */
int vh_slice_csr(const void* data, int32_t dtype, const int32_t* indices, const int32_t* indptr, int64_t rows,
                 int64_t cap, int32_t dim, int64_t start, int64_t end, int64_t out_cap, void* out_data,
                 int32_t* out_indices, int32_t* out_indptr, vh_stream_t stream);

/* spmm_csr (ops/quantized.py:1567-1645): for each of `batch` CSR matrices
 * ([rows, K], `cap` slots; row pointers rebased on their first, clamped to
 * [0, cap] and made non-decreasing as the reference's cummax; columns
 * clamped to [0, K - 1]) times the dense B (b_layout 0: "kc", stored
 * [N, K]; 1: "ck", stored [K, N]; b_batch_stride elements between batches,
 * 0: one B for all), out[b, r, n] = sum over the row's entries, in order,
 * of float32(data) * float32(B[k, n]), plus base[b, r, n] (float32,
 * optional: the GEMM product it adds to), rounded once to out_dtype.
 * work: int32 [batch, rows + 1] for the rebased row pointers. */
int vh_spmm_csr(const void* data, int32_t data_dtype, const int32_t* indices, const int32_t* indptr, int64_t batch,
                int64_t rows, int64_t cap, const void* B, int32_t b_dtype, int32_t b_layout, int64_t K, int64_t N,
                int64_t b_batch_stride, const float* base, void* out, int32_t out_dtype, int32_t* work,
                vh_stream_t stream);

/* ------------------------------------------------------------ conv2d
 * quantized_ops.conv2d (ops/layout.py:170-215) and the convolution of
 * conv2d_mx (ops/quantized.py:596-643) as im2col + vh_gemm: per group, A
 * [N*OH*OW, kp] holds each output pixel's input patch (columns (c, kh, kw)
 * of the group's channels, zero past Cg*KH*KW), B [K/groups, kp] the
 * group's filters in the same column order; vh_gemm writes the group's
 * output channels of an NHWC result, vh_nhwc_to_nchw transposes it for an
 * NCHW layout.  Feature maps NCHW or NHWC (nhwc != 0); weights OIHW, or
 * HWIO (hwio != 0, dense convolutions only). */
typedef struct vh_conv_geom {
  int64_t N, C, H, W; /* input */
  int64_t K, KH, KW;  /* output channels, filter size */
  int64_t OH, OW;     /* output size (must follow from the rest, as aten computes it) */
  int32_t stride[2], padding[2], dilation[2];
  int32_t groups;
} vh_conv_geom;

int vh_conv_im2col(const void* x, int32_t dtype, const vh_conv_geom* geom, int32_t nhwc, int32_t group, int64_t kp,
                   void* a, vh_stream_t stream);
int vh_conv_pack_weight(const void* w, int32_t dtype, const vh_conv_geom* geom, int32_t hwio, int32_t group,
                        int64_t kp, void* out, vh_stream_t stream);
/* dst [n, c, p] = src [n, p, c] (bf16, fp16 or fp32). */
int vh_nhwc_to_nchw(const void* src, int32_t dtype, int64_t n, int64_t p, int64_t c, void* dst, vh_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* VOYAGER_HIP_H */
