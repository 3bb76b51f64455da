/* vybdq.h — MI355X (gfx950) fused dequant-matmul library: flat C-ABI.
 *
 * Buffer-in / buffer-out. Every device buffer is a plain device address passed as
 * uint64_t (the reference host keeps device pointers as Int handles,
 * native/tensor/tensor.vyb:11-22). Streams are hipStream_t handles passed as uint64_t
 * (0 = the null stream). The caller allocates and owns every buffer; no entry point
 * allocates or frees device memory inside a hot call, and none synchronises the stream.
 *
 * Return codes: 0 = success; a negative VYBDQ_ERR_* code otherwise, with the message in
 * vybdq_last_error() (per host thread). Shape preconditions are checked before any launch
 * (the reference's EXL3FAIL checks, native/glm53/glm_engine.vyb:969-973). No scalar
 * out-parameters (native/audio/vyb_audio.h:25-28): sizes are returned as int64_t.
 *
 * Packed formats (little-endian, GGUF row layout: weight row n = output n, K/32 blocks):
 *   q4_0: 18 B = [fp16 d][16 B nibbles], w = d * (q - 8)
 *   Q8_0: 34 B = [fp16 d][32 x int8],    w = d * q
 *   EXL3 4-bpw: trellis uint16 [K/16][N/16][64], suh fp16 [K], svh fp16 [N]
 * GGUF K-quant super-blocks (256 weights, rows are K/256 super-blocks; llama.cpp layouts):
 *   Q4_K: 144 B = [fp16 d][fp16 dmin][scales 12 B: 6-bit sc, m per 32][qs 128 B]
 *   Q5_K: 176 B = [fp16 d][fp16 dmin][scales 12 B][qh 32 B][qs 128 B]
 *   Q6_K: 210 B = [ql 128 B][qh 64 B][int8 scales per 16][fp16 d]
 * Results are deterministic: fixed reduction order, no floating-point atomics.
 */
#ifndef VYBDQ_H
#define VYBDQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VYBDQ_ABI_VERSION 1

/* return codes */
#define VYBDQ_OK 0
#define VYBDQ_ERR_ARG (-1)       /* null pointer, unknown enum value */
#define VYBDQ_ERR_SHAPE (-2)     /* shape precondition failed; nothing was launched */
#define VYBDQ_ERR_ALIGN (-3)     /* buffer alignment precondition failed */
#define VYBDQ_ERR_HIP (-4)       /* HIP runtime error (launch failure etc.) */
#define VYBDQ_ERR_WORKSPACE (-5) /* workspace missing or too small */

/* element types (x_dt / y_dt / out_dt) */
#define VYBDQ_F32 0
#define VYBDQ_F16 1
#define VYBDQ_BF16 2
#define VYBDQ_F64 3

/* q4_0 nibble order within a block */
#define VYBDQ_Q4_GGML 0        /* element j = low nibble of qs[j], j+16 = high nibble (GGUF) */
#define VYBDQ_Q4_INTERLEAVED 1 /* element 2s = low, 2s+1 = high nibble of qs[s]; the order of
                                  the reference's deq_q4_0 intrinsic, pinned by its fixture
                                  (native/gguf/mk_fixture.vyb:86-99, dequant_gguf.vyb:118-127) */

/* EXL3 codebook (exllamav3 numbering). mcg, x = w*0xCBAC1FED, is exllamav3's decode_3inst at
   cb=1 and the only codebook the reference implements (native/exl3/exl3_ref.py:19-22,
   native/kernels/exl3.vyb:15-19); every EXL3 entry point returns VYBDQ_ERR_ARG for any other
   value (codebook 0, QTIP's multiply-add 3INST, and codebook 2, mul1, are not supported). */
#define VYBDQ_EXL3_MCG 1

/* ---- library ------------------------------------------------------------------------- */

/* VYBDQ_ABI_VERSION of the loaded library. */
int vybdq_abi_version(void);

/* Text of the failure from the last vybdq_* call on this host thread that failed.
   Never NULL. Mirrors va_lasterr (native/audio/vyb_audio.h:16-19). */
const char *vybdq_last_error(void);

/* ---- decode-only entry points (the bit-exact gates) ---------------------------------- */

/* out[i] = d * (q - 8) for nblocks*32 elements; out_dt F32, F16 or F64.
   Replaces q4deq(q, o, n, z) (native/kernels/deq.vyb:4-12), which writes f64. */
int vybdq_dequant_q4_0(uint64_t W, uint64_t out, int64_t nblocks, int order, int out_dt,
                       uint64_t stream);

/* out[i] = d * q for nblocks*32 elements; out_dt F32, F16 or F64.
   Replaces q8_0deq(q, o, n, z=0) (native/kernels/q8_0.vyb:11-30). */
int vybdq_dequant_q8_0(uint64_t W, uint64_t out, int64_t nblocks, int out_dt, uint64_t stream);

/* out[i] = weight i of n consecutive weights of type wtype (GGML type id: 2 = q4_0 in GGUF
   order, 8 = Q8_0, 12 = Q4_K, 13 = Q5_K, 14 = Q6_K, 22 = IQ2_S); n % 32 == 0 (super-block types:
   n % 256 == 0);
   out_dt F32, F16 or F64 (F64: exact; F32: the exact value rounded once; F16: the F32 rounded).
   Replaces q4kdeq / q4kdeq32 (native/kernels/q4k.vyb:9-70) and the q5_K / q6_K decodes the
   reference gates (native/tools/q5k_ref.py:40-65, native/gguf/q6k_verify.py:20-40). */
int vybdq_dequant(int wtype, uint64_t W, uint64_t out, int64_t n, int out_dt, uint64_t stream);

/* ---- GEMV on packed GGUF rows -------------------------------------------------------- */

/* The GEMV below for any GGUF weight type, dispatched on the GGML type id as the reference's
   gemv_h(ty) does (native/host/ridge_decode.vyb:303-311): 2 = q4_0 (GGUF nibble order), 8 = Q8_0,
   12 = Q4_K, 13 = Q5_K, 14 = Q6_K, 22 = IQ2_S. Super-block types need K % 256 == 0 and W 4-byte
   aligned. Replaces gemv_iq2s (native/kernels/rgemv.vyb:24-80),
   gemv_q4k (native/kernels/qwen3.vyb:403-576), gemv_q6k (qwen3.vyb:726-887) and gemv_q5k
   (native/kernels/rgemv.vyb:202-297), p-block W@0 X@8 Y@16 N@32 K@40 YE@48 RS@120. */
int vybdq_gemv(int wtype, uint64_t W, uint64_t X, uint64_t Y, int64_t M, int64_t N, int64_t K,
               int x_dt, int y_dt, uint64_t RS, uint64_t stream);


/* Y[m, n] = RS[m, n] + sum_k X[m, k] * W[n, k] for m < M, n < N.
   X: x_dt (F32, F16, BF16) [M, K]; Y: y_dt (F32, F16, BF16, F64) [M, N]; RS: same type as
   Y or 0. K % 32 == 0; 1 <= M <= 8. Accumulation in float32. Every GEMV entry point (and the
   MoE layer's expert GEMV up to 64 tokens) stages X as fp16 per 32-element block: F32 / BF16 X
   is first scaled by the power of two that brings the block's largest |x| into [2^14, 2^15)
   (folded back into the block's weight scale), so activations of any magnitude neither overflow
   nor flush to zero; F32 values are rounded to fp16 (11 significant bits) at staging.
   Replaces gemv_q8_0's sibling for q4_0 (p-block W@0 X@8 Y@16 M@24 N@32 K@40 YE@48 RS@120,
   native/kernels/rgemv.vyb:13-15, native/kernels/qwen3.vyb:395-440); the reference has no
   fused q4_0 GEMV, only deq_q4_0 followed by the f64 gemm (native/kernels/gemm.vyb:15-39). */
int vybdq_gemv_q4_0(uint64_t W, uint64_t X, uint64_t Y, int64_t M, int64_t N, int64_t K,
                    int x_dt, int y_dt, uint64_t RS, int order, uint64_t stream);

/* Same contract on Q8_0 rows. Replaces gemv_q8_0 (native/kernels/rgemv.vyb:299-368). */
int vybdq_gemv_q8_0(uint64_t W, uint64_t X, uint64_t Y, int64_t M, int64_t N, int64_t K,
                    int x_dt, int y_dt, uint64_t RS, uint64_t stream);

/* Fused launch of up to three q4_0 GEMVs that share X (q|k|v, gate|up): rows [0, N) go to
   W/Y, the next N2 rows to W2/Y2, the next N3 to W3/Y3 (N2 = N3 = 0: one matrix). Mirrors
   the multi-segment p-block (W2/NS2/Y2/YE2 @56-80, W3/NS3/Y3/YE3 @88-112,
   native/kernels/qwen3.vyb:416-436). M = 1. */
int vybdq_gemv_q4_0_seg3(uint64_t X, int64_t K, int x_dt, int order,
                         uint64_t W, uint64_t Y, int64_t N, int y_dt,
                         uint64_t W2, uint64_t Y2, int64_t N2, int y_dt2,
                         uint64_t W3, uint64_t Y3, int64_t N3, int y_dt3, uint64_t stream);

/* Fused launch of up to three GEMVs of GGUF type wtype (2, 8, 12, 13, 14, 22 as vybdq_gemv) that
   share X [M, K] (M <= 8): segment i has N_i rows W_i -> Y_i [M, N_i] of y_dt_i, plus its optional
   residual RS_i of the same type; a segment with N_i = 0 is absent (its pointers are ignored).
   Mirrors the multi-segment p-block of gemv_q4k / gemv_q6k, which fuses q|k|v and gate|up
   (W2/NS2/Y2/YE2 @56-80, W3/NS3/Y3/YE3 @88-112, RS@120, native/kernels/qwen3.vyb:416-436), and the
   two Q8_0 matrices of one gemv_q8_0_sk launch (p and p+256, native/kernels/rq80s.vyb:1-12):
   one launch, X staged once. */
int vybdq_gemv_seg3(int wtype, uint64_t X, int64_t M, int64_t K, int x_dt,
                    uint64_t W, uint64_t Y, int64_t N, int y_dt, uint64_t RS,
                    uint64_t W2, uint64_t Y2, int64_t N2, int y_dt2, uint64_t RS2,
                    uint64_t W3, uint64_t Y3, int64_t N3, int y_dt3, uint64_t RS3, uint64_t stream);

/* Decode GEMV on an xq8 activation row: Y[n] = RS[n] + sum_k W[n, k] * x'[k] with
   x'[k] = Xs[k / 32] * Xq[k] (Xq int8 [K], Xs float32 [K/32]: the layout vybdq_quant_q8_act,
   vybdq_rmsnorm_q8 and vybdq_swiglu_q8 write; the reference keeps both in one buffer, Xs = Xq + K).
   wtype 12 (Q4_K), 13 (Q5_K) or 22 (IQ2_S). Every 32-weight sub-block product is an exact integer
   dot product, scaled and accumulated in float32: the result matches the float64 GEMV of x' to
   float32 rounding, and differs from the exact entry points (vybdq_gemv on x) by the activation
   quantization, which the reference accepts on its default decode path (doc/RIDGE-27B.md:75-84).
   K % 256 == 0, K <= 65536; Xq 16-byte and Xs 4-byte aligned; W 4-byte aligned; y_dt F32, F16,
   BF16 or F64, RS of the same type or 0. Replaces gemv_iq2s_q (p-block W@0 X@8 Y@16 N@32 K@40
   YE@48 RS@120 G@128, native/kernels/rgemv7.vyb:3-96), gemv_q4k_q / gemv_q4k_qu
   (native/kernels/rq4kq.vyb:7-89,93-274) and gemv_q5k_q / gemv_q5k_qu
   (native/kernels/rq5kq.vyb:8-80,82-268); the IQ2_S grid is built in. */
int vybdq_gemv_xq8(int wtype, uint64_t W, uint64_t Xq, uint64_t Xs, uint64_t Y, int64_t N, int64_t K,
                   int y_dt, uint64_t RS, uint64_t stream);

/* vybdq_gemv_xq8 over up to three matrices sharing the xq8 row (segments as vybdq_gemv_seg3),
   one launch: the multi-segment block of gemv_q4k_q / gemv_q5k_q (W2/NS2/Y2/YE2 @56-80,
   W3/NS3/Y3/YE3 @88-112, native/kernels/rq4kq.vyb:18-33). */
int vybdq_gemv_xq8_seg3(int wtype, uint64_t Xq, uint64_t Xs, int64_t K,
                        uint64_t W, uint64_t Y, int64_t N, int y_dt, uint64_t RS,
                        uint64_t W2, uint64_t Y2, int64_t N2, int y_dt2, uint64_t RS2,
                        uint64_t W3, uint64_t Y3, int64_t N3, int y_dt3, uint64_t RS3, uint64_t stream);

/* Router logits Y [T, E] = X [T, H] W^T with W [E, H] (w_dt F32, F16 or BF16; the checkpoint's
   router weight is bf16), X of x_dt (F32, F16, BF16 or F64), accumulated in float64 (every
   product exact; fixed lane-strided order); y_dt F64 or F32. vybdq_moe_route / vybdq_moe_forward
   take F64 logits as they are. Replaces the router GEMM of native/glm53/glm_engine.vyb:2728-2745
   (deq_bf16 to float64, then a float64 matmul). */
int vybdq_router_logits(uint64_t X, int x_dt, uint64_t W, int w_dt, uint64_t Y, int y_dt, int64_t T,
                        int64_t E, int64_t H, uint64_t stream);

/* ---- producer-side q8 activation quantization ---------------------------------------- */

/* Per row of X [M, N]: y = x * r * w with r = 1 / sqrt(sum x^2 / N + eps), in float64 with the
   reference's summation order and seeded-Newton square root; writes any of Y [M, N] (y_dt),
   Y32 [M, N] float32 and the q8 copy of the float32 values (Xq int8 [M, N], Xs float32
   [M, N/32], N % 32 == 0; xq8 semantics). X and W [N] have element type x_dt (F64, F32, F16,
   BF16). Replaces rms_blkg with its Y32 and Y8 outputs (native/kernels/layer.vyb:989-1066,
   VYB_RMSQ8); the reference's single Y8 buffer is Xq followed by Xs (M = 1). */
int vybdq_rmsnorm_q8(uint64_t X, uint64_t W, uint64_t Y, uint64_t Y32, uint64_t Xq, uint64_t Xs,
                     int64_t M, int64_t N, double eps, int x_dt, int y_dt, uint64_t stream);

/* h = g * sigmoid(g) * u elementwise in float64 with the reference's exp (vmath.vyb:7-40);
   writes H [n] (h_dt, F32 in the reference) and/or the q8 copy of float32(h) (Xq, Xs;
   n % 32 == 0). G and U have element type g_dt (F64, F32, F16, BF16). Replaces silu32q
   (native/kernels/layer.vyb:1567-1590, VYB_SWQ8). */
int vybdq_swiglu_q8(uint64_t G, uint64_t U, uint64_t H, uint64_t Xq, uint64_t Xs, int64_t n, int g_dt,
                    int h_dt, uint64_t stream);

/* ---- GGUF reader and packed-slab residency (host) ------------------------------------ */

/* Opens and indexes a GGUF v2/v3 file (header, every metadata pair, every tensor info); returns
   a handle >= 1 or a negative error code. Replaces the reference's Vyb readers
   (native/gguf/parse_gguf.vyb, native/gguf/read_real_meta.vyb). */
int64_t vybdq_gguf_open(const char *path);
int vybdq_gguf_close(int64_t h);
/* what: 0 version, 1 tensor count, 2 metadata count, 3 alignment, 4 end of the tensor infos,
   5 data section start (4 rounded up to the alignment), 6 file size. */
int64_t vybdq_gguf_info(int64_t h, int what);
/* index of the tensor / metadata pair with that name, -1 if absent */
int64_t vybdq_gguf_find_tensor(int64_t h, const char *name);
int64_t vybdq_gguf_find_kv(int64_t h, const char *key);
/* copies the name (NUL-terminated, at most cap - 1 bytes) and returns its full length */
int64_t vybdq_gguf_tensor_name(int64_t h, int64_t i, char *buf, int64_t cap);
/* what: 0 ggml type, 1 n_dims, 2 + d dims[d], -1 the raw offset field, -2 data bytes
   (-1 for a type this library does not size) */
int64_t vybdq_gguf_tensor_field(int64_t h, int64_t i, int what);
int64_t vybdq_gguf_kv_key(int64_t h, int64_t i, char *buf, int64_t cap);
/* what: 0 value type, 1 integer value (integer and bool types), 2 array element type,
   3 array length */
int64_t vybdq_gguf_kv_field(int64_t h, int64_t i, int what);
/* float value of a f32 / f64 pair (integers converted; 0.0 for a bad handle or index) */
double vybdq_gguf_kv_float(int64_t h, int64_t i);
int64_t vybdq_gguf_kv_string(int64_t h, int64_t i, char *buf, int64_t cap);
/* Reads tensor i's bytes into host memory (cap >= its size); absolute = 1 takes the offset
   field as a file offset (the convention of the reference's fixture writer,
   native/gguf/mk_fixture.vyb), 0 as relative to the data section (the GGUF convention).
   Returns the byte count. */
int64_t vybdq_gguf_read_tensor(int64_t h, int64_t i, int absolute, void *dst, int64_t cap);
/* One-buffer residency (the reference's resident packed slab, native/host/ridge_decode.vyb:1-3):
   every tensor in index order at an offset rounded up to align (a power of two). */
int64_t vybdq_gguf_slab_offset(int64_t h, int64_t i, int64_t align);
int64_t vybdq_gguf_slab_bytes(int64_t h, int64_t align);
/* Copies every tensor into the device slab dev (dev_bytes >= vybdq_gguf_slab_bytes) on stream
   through a host buffer; returns when the copies have finished. */
int vybdq_gguf_load_slab(int64_t h, uint64_t dev, int64_t dev_bytes, int64_t align, int absolute,
                         uint64_t stream);

/* ---- safetensors reader and sharded-checkpoint index (host) ------------------------- */

/* Opens and indexes a safetensors file (u64 LE header length, JSON header, data region): every
   tensor's dtype, shape and byte range (checked against the file and, for the sized dtypes,
   against shape x element size) and the __metadata__ strings. Returns a handle >= 1 or a
   negative error code. Replaces native/torchload/safetensors.vyb (container layout :8-19,
   dtype table :48-66). */
int64_t vybdq_st_open(const char *path);
int vybdq_st_close(int64_t h);
/* what: 0 tensor count, 1 metadata count, 2 header length, 3 data region start, 4 file size */
int64_t vybdq_st_info(int64_t h, int what);
/* tensor index (header order) of name, -1 if absent */
int64_t vybdq_st_find(int64_t h, const char *name);
/* copy the name / dtype spelling (NUL-terminated, at most cap - 1 bytes); return full length */
int64_t vybdq_st_tensor_name(int64_t h, int64_t i, char *buf, int64_t cap);
int64_t vybdq_st_tensor_dtype(int64_t h, int64_t i, char *buf, int64_t cap);
/* what: 0 element size (0 for a dtype not sized here), 1 ndim, 2 + d shape[d], -1 absolute file
   offset of the data, -2 data bytes */
int64_t vybdq_st_tensor_field(int64_t h, int64_t i, int what);
/* __metadata__ value for key (full length), -1 if absent */
int64_t vybdq_st_meta(int64_t h, const char *key, char *buf, int64_t cap);
/* key of metadata pair i (header order; full length) */
int64_t vybdq_st_meta_key(int64_t h, int64_t i, char *buf, int64_t cap);
/* tensor i's bytes into host memory (cap >= its size); returns the byte count */
int64_t vybdq_st_read(int64_t h, int64_t i, void *dst, int64_t cap);
/* tensor i's bytes into device memory dev (dev_bytes >= its size), ordered on stream; returns the
   byte count after the copies have finished */
int64_t vybdq_st_upload(int64_t h, int64_t i, uint64_t dev, int64_t dev_bytes, uint64_t stream);
/* model.safetensors.index.json: tensor name -> shard file through "weight_map" (the name -> shard
   step of native/glm53/gx.vyb:1-16). */
int64_t vybdq_st_index_open(const char *path);
int vybdq_st_index_close(int64_t h);
int64_t vybdq_st_index_count(int64_t h);
/* entry i (file order): copies the tensor name and its shard file; returns the name's full length */
int64_t vybdq_st_index_entry(int64_t h, int64_t i, char *name, int64_t name_cap, char *shard, int64_t shard_cap);
/* shard file of a tensor (full length), -1 if the index does not list it */
int64_t vybdq_st_index_shard(int64_t h, const char *name, char *buf, int64_t cap);

/* ---- persistent chain of dependent GEMV stages --------------------------------------- */

/* Bytes of workspace vybdq_gemv_chain needs for nstages stages (a status word and one counter
   per stage). Zero-fill it once before the first call; a completed call leaves it zero-filled. */
int64_t vybdq_chain_workspace_size(int nstages);

/* Run nstages dependent GEMV stages in ONE persistent launch. Stage s is described by the
   reference's GEMV parameter block at device address P + s*pstride (W@0 X@8 Y@16 M@24 N@32
   K@40 YE@48 W2@56 NS2@64 Y2@72 YE2@80 W3@88 NS3@96 Y3@104 YE3@112 RS@120 GRID@128,
   native/host/ridge_decode.vyb:264-270) plus XE@136 (x type: 2 = f16, 258 = bf16, else f32)
   and ORDER@144 (q4_0 nibble order). YE: 4 = f32, 2 = f16, 258 = bf16, else f64 with the f64
   residual RS (the reference's YE rule, rgemv.vyb:13-15). M must be 1; K % 64 == 0, K <= max_K.
   Stage s computes only after every workgroup finished stage s-1, so its X may be stage s-1's
   Y; its weights are prefetched before that wait. wtype: 2 = q4_0, 8 = Q8_0 (GGUF type ids).
   Replaces a sequence of lk(gemv, grid, 512, p) launches (ridge_decode.vyb:204-227). */
int vybdq_gemv_chain(int wtype, uint64_t P, int nstages, int64_t pstride, int64_t max_K, uint64_t ws,
                     uint64_t stream);

/* Synchronous check of a chain workspace after the stream is idle: 0, or an error if a stage
   wait timed out or a stage descriptor was invalid in a previous call. */
int vybdq_chain_status(uint64_t ws);

/* ---- EXL3 4-bpw trellis ------------------------------------------------------------- */

/* Rotated-basis decode What [K, N] (no Hadamard, no scales); out_dt F32, F16 or F64. The
   bit-exact gate: replaces exl3deq / exl3deq32 (native/kernels/exl3.vyb:207-242,375-422),
   with the tile-slot composition built in (native/exl3/tile_slot_composition.json). */
int vybdq_exl3_decode_tiles(uint64_t trellis, uint64_t out, int64_t K, int64_t N, int codebook,
                            int out_dt, uint64_t stream);

/* Full original-basis W [K, N] = diag(suh) (H/sqrt128) What (H/sqrt128) diag(svh), per 128x128
   block, float32 transforms; out_dt F32, F16 or F64; K, N % 128 == 0. Replaces the exl3_deq32
   pipeline exl3dq1s + exl3had232 + exl3cvt32 (native/glm53/glm_engine.vyb:1103-1200,
   native/kernels/exl3dq.vyb:46-113). */
int vybdq_dequant_exl3(uint64_t trellis, uint64_t suh, uint64_t svh, uint64_t out, int64_t K, int64_t N,
                       int codebook, int out_dt, uint64_t stream);

/* Workspace bytes for vybdq_exl3_gemm at (B, K, N), or -1 for an unsupported shape. */
int64_t vybdq_exl3_workspace_size(int64_t B, int64_t K, int64_t N);

/* Y [B, N] = X [B, K] W, W the EXL3 matrix above, without materialising W: X is rotated
   (FWHT(X * suh)/sqrt128 per 128 chunk), the trellis is decoded in registers and multiplied
   (f32 accumulation), and the result rotated back (FWHT(.)/sqrt128 * svh). 1 <= B <= 16,
   K, N % 128 == 0, trellis 16-byte aligned, ws 256-byte aligned of at least
   vybdq_exl3_workspace_size bytes, zero-filled once before the first call (it holds arrival
   counters that every completed call leaves at zero; calls sharing a workspace must not run
   concurrently). One kernel launch for B <= 2, three above. The reference has no fused EXL3 GEMM (it dequantizes each
   expert to f64/f32 then runs gemm, glm_engine.vyb:2845-2923). */
int vybdq_exl3_gemm(uint64_t trellis, uint64_t suh, uint64_t svh, uint64_t X, uint64_t Y, int64_t B,
                    int64_t K, int64_t N, int codebook, int x_dt, int y_dt, uint64_t ws, int64_t ws_bytes,
                    uint64_t stream);

/* ---- prefill / grouped dequant GEMM ----------------------------------------------------- */

/* Y [M, N] (row stride ldy, 0 = N) = X [M, K] W^T (+ RS) with W packed GGUF rows of type wtype
   (2 = q4_0 GGUF order, 8 = Q8_0, 12 = Q4_K, 13 = Q5_K, 14 = Q6_K, 22 = IQ2_S): weights are
   dequantized to fp16 (q4_0 / Q8_0: d * (q - OFF), one rounding; super-block types: the exact
   value rounded to float32, then to fp16, as vybdq_dequant's F16 output) and multiplied with fp16
   MFMA, float32 accumulation; X (f32/f16/bf16) is converted to fp16 as it is (|x| < 65504, as
   the reference's f16 tiles require; vybdq_gemm_ws lifts this).
   q4_0 / Q8_0: K % 64 == 0; M >= 64 with K % 256 == 0 and N % 16 == 0 runs the kernel that
   dequantizes into the MFMA operand registers; other shapes need N % 64 == 0 and stage the
   dequantized tile in LDS. Super-block types: K % 256 == 0, N % 64 == 0, any M. Q4_K with
   M >= 64, K < 2^22 and fp16 X (any X type through vybdq_gemm_ws) dequantizes into the operand
   registers too, each weight as one fp16 fma q * fp16(d sc) - fp16(dmin m) (within one fp16 ulp
   of the weight's scale of the F16 dequant value). Q6_K and IQ2_S with M >= 96 and fp16 or
   bf16 X (f32 X through vybdq_gemm_ws) run 128-row tiles whose weights are formed in fp16
   arithmetic: fp16(d sc) * (q - 32), fp16(d (0.5 + s) / 4) * grid magnitude (one product
   rounding after the rounding of the scale); so do Q4_K and Q5_K with bf16 X from 96 rows
   (fp16(d sc) * q - fp16(dmin m), as the register body).
   Replaces gemm_q80 and its siblings picked by gemm_h(ty) (native/host/ridge_decode.vyb:295-302,
   native/tools/gen_rpf.py:1-10,142-149, p-block W@0 X@8 Y@16 S@24 N@32 K@40 LDY@48 RS@56). */
int vybdq_gemm(int wtype, uint64_t W, uint64_t X, uint64_t Y, int64_t M, int64_t N, int64_t K, int x_dt,
               int y_dt, int64_t ldy, uint64_t RS, uint64_t stream);

/* Workspace bytes vybdq_gemm_ws can use at (M, N, K) (q4_0, Q8_0, Q4_K, Q5_K from 64 rows; Q6_K,
   IQ2_S from 96 rows): split-K partials and the fp16 copy of a bf16/f32 X; 0 when the shape does
   not use the workspace. */
int64_t vybdq_gemm_workspace_size(int wtype, int64_t M, int64_t N, int64_t K);

/* vybdq_gemm with a caller workspace ws (256-byte aligned, ws_bytes, any contents; 0 = none). With
   a workspace of at least vybdq_gemm_workspace_size bytes, long-K shapes split K across
   workgroups: each stores float32 partials and a second kernel sums them in split order, so
   results stay deterministic for a fixed shape and workspace (they may differ in the last bits
   from the unsplit vybdq_gemm); bf16/f32 X is converted to fp16 once into the workspace instead of
   once per output tile, each row scaled by the power of two that brings its largest |x| into
   [2^14, 2^15) (multiplied back into the row's outputs), so X of any magnitude neither overflows nor
   flushes to zero. Calls that share a workspace must not overlap. The reference's gemm_q80
   has no workspace (native/tools/gen_rpf.py:58-62); this is the same GEMM for shapes whose
   tiles alone do not fill the GPU. */
int vybdq_gemm_ws(int wtype, uint64_t W, uint64_t X, uint64_t Y, int64_t M, int64_t N, int64_t K, int x_dt,
                  int y_dt, int64_t ldy, uint64_t RS, uint64_t ws, int64_t ws_bytes, uint64_t stream);

/* Workspace bytes vybdq_gemm_q8_0_i8 can use at (M, N, K) to split K across workgroups, 0 when the
   shape gains nothing from a split. */
int64_t vybdq_gemm_q8_0_i8_workspace_size(int64_t M, int64_t N, int64_t K);

/* int8 path. Y [M, N] (row stride ldy, 0 = N) = RS + sum_b Xs[m, b] * d[n, b] * (Xq[m, b] . q[n, b])
   over the 32-element blocks b, with Xq int8 [M, K] and Xs float32 [M, K/32] as written by
   vybdq_quant_q8_act (xq8 semantics) and W packed Q8_0 rows (d fp16, q int8). Each block product
   is an exact int32 MFMA; scaling and accumulation are float32. K % 256 == 0, N % 16 == 0; W, Xq and
   Xs 16-byte aligned; ws / ws_bytes as for vybdq_gemm_ws (sized by
   vybdq_gemm_q8_0_i8_workspace_size). The reference quantizes activations with xq8 and runs
   q8_1 x Q8_0 dot-product GEMVs (native/kernels/rgemv7.vyb:195-214, native/tools/gen_rgemv7.py:1-8);
   this is the same arithmetic as a prefill GEMM. */
int vybdq_gemm_q8_0_i8(uint64_t W, uint64_t Xq, uint64_t Xs, uint64_t Y, int64_t M, int64_t N, int64_t K, int y_dt,
                       int64_t ldy, uint64_t RS, uint64_t ws, int64_t ws_bytes, uint64_t stream);

/* ---- the reference's own parameter blocks ------------------------------------------------ */

/* kind of a parameter block: GEMV / GEMM kinds plus the GGML type id of W (2, 8, 12, 13, 14, 22);
   the MoE and EXL3 kinds take no type id */
#define VYBDQ_PB_GEMV 0x100     /* set_gemv layout (the packed GEMV kernels) */
#define VYBDQ_PB_GEMM 0x200     /* set_gemm layout, X float32 (the gen_rpf prefill tiles) */
#define VYBDQ_PB_GEMM_XH 0x300  /* set_gemm layout, X fp16 (the gen_rpf --xh tiles) */
#define VYBDQ_PB_MOE 0x400      /* moe_route + moe_act + moe_down block (native/kernels/moe.vyb) */
#define VYBDQ_PB_EXL3DQ 0x500   /* exl3dq1 / exl3dq1s block (exl3.vyb, exl3dq.vyb); needs the grid */
#define VYBDQ_PB_EXL3INV 0x600  /* exl3inv block (exl3.vyb) */
#define VYBDQ_PB_EXL3HGEN 0x700    /* exl3hgen block (exl3.vyb:36-56): H float64 */
#define VYBDQ_PB_EXL3HGEN32 0x701  /* exl3hgen32 block (exl3.vyb:124-145): H float32 */
#define VYBDQ_PB_EXL3HAD1 0x800    /* exl3had1 block (exl3.vyb:58-86): column transform, float64 */
#define VYBDQ_PB_EXL3HAD132 0x801  /* exl3had132 block (exl3.vyb:147-172): column transform, float32 */
#define VYBDQ_PB_EXL3HAD2 0x900    /* exl3had2 block (exl3.vyb:88-118): row transform + scales, float64 */
#define VYBDQ_PB_EXL3HAD232 0x901  /* exl3had232 block (exl3.vyb:174-202): row transform + scales, float32 */
#define VYBDQ_PB_EXL3CVT32 0xA00   /* exl3cvt32 block (exl3.vyb:247-256): float32 -> float64 */

/* Launch one GEMV or prefill GEMM described by a reference parameter block at device address P
   (8-byte aligned): little-endian int64 words, each read by the kernel when the launch runs (the
   reference rewrites block words with asynchronous copies inside its captured decode graph,
   native/host/ridge_decode.vyb:168-180), so the host reads nothing and the call can be captured.
   Replaces lk(h, gx, bx, p) (ridge_decode.vyb:204-227) with h picked by gemv_h / gemm_h (:295-311).
   VYBDQ_PB_GEMV + ty, set_gemv (ridge_decode.vyb:264-270): W@0 X@8 Y@16 M@24 N@32 K@40 YE@48
     W2@56 NS2@64 Y2@72 YE2@80 W3@88 NS3@96 Y3@104 YE3@112 RS@120 (GRID@128 unused): up to three
     row segments sharing x f32 [K]; M must be 1; YE = 4: f32 output, otherwise f64 output plus the
     f64 residual RS (segment 1); K % 64 == 0 (super-block types K % 256 == 0), K <= 20480;
     W 4-byte and X 16-byte aligned.
   VYBDQ_PB_GEMM / VYBDQ_PB_GEMM_XH + ty, set_gemm (ridge_decode.vyb:272-275, native/tools/gen_rpf.py:2-8):
     W@0 X@8 Y@16 S@24 N@32 K@40 LDY@48 RS@56 (G@64, NMT@72 unused): Y[s, n] = RS[s, n] +
     sum_k X[s, k] W[n, k] for s < S; LDY >= N: Y float64 of row stride LDY, RS float64 or 0;
     LDY <= -N: Y float32 of row stride -LDY, RS ignored; K % 256 == 0; N % 16 == 0 (q4_0 / Q8_0) or
     N % 64 == 0 (super-block types); no K split (the block has no workspace word).
   VYBDQ_PB_MOE, moe.vyb:15-19 (replaces the three launches of moe_driver.vyb:150-159):
     y@0 G@8 bias@16 LG@24 IX@32 WT@40 AC@48 wg_e@56 wu_e@64 wd_e@72 wg_s@80 wu_s@88 wd_s@96
     out@104 S@112; fixed H = 4096, I = 2048, 288 experts, top-8, dense float32 weights [in][out];
     1 <= S <= 256; writes LG [S][288], IX [S][8] (expert ids as floats), WT [S][8],
     AC [S][9][2048] and out [S][4096]; y, G, AC 16-byte and the other buffers 4-byte aligned.
   VYBDQ_PB_EXL3INV, exl3.vyb:318-333: td@0 nbody@8; writes the inverse tile map
     (u32 [256] at td + 16 + nbody).
   The stages of the reference's separate EXL3 reconstruction (glm_engine.vyb:1103-1200,
   native/host/glm_exl3_check32.vyb:150-240), T = float64 for HGEN / HAD1 / HAD2 and float32 for
   the *32 kinds; every buffer 16-byte aligned except suh / svh (2-byte):
   VYBDQ_PB_EXL3HGEN / HGEN32: H@0; writes H T [128][128] = (-1)^popcount(i & j) *
     T(0.08838834764831845).
   VYBDQ_PB_EXL3HAD1 / HAD132: W@0 Tmp@8 H@16 cw@24 nbc@32 nblocks@40; for each block
     = kb nbc + nb < nblocks: Tmp[block][b][d] = sum over c ascending of
     W[(128 kb + b) cw + 128 nb + c] H[c][d] (fma chain); nbc >= 1, cw >= 128 nbc, cw a multiple
     of 4 (float32) or 2 (float64).
   VYBDQ_PB_EXL3HAD2 / HAD232: Tmp@0 O@8 H@16 suh@24 svh@32 cw@40 nbc@48 nblocks@56;
     O[(128 kb + a) cw + 128 nb + d] = (sum over b ascending of H[a][b] Tmp[block][b][d])
     * T(suh[128 kb + a]) * T(svh[128 nb + d]) (suh, svh fp16).
   VYBDQ_PB_EXL3CVT32: S@0 D@8 n@16; D float64 [n] = S float32 [n] (S 4-, D 8-byte aligned).
   A block whose words violate these is not computed (nothing is written) and the next
   vybdq_pblock_status() on the device reports it; the call itself only checks kind and P. */
int vybdq_launch_pblock(int kind, uint64_t P, uint64_t stream);

/* vybdq_launch_pblock with the reference launch's grid (grid_x blocks of block_x threads), for
   kinds whose extent is the thread count rather than a block word; other kinds ignore the grid.
   Replaces cuda_launch4i(f, grid_x, 1, 1, block_x, 1, 1, p) (native/host/moe_driver.vyb:20).
   VYBDQ_PB_EXL3DQ, exl3.vyb:264 / exl3dq.vyb:8-11: q@0 td@8 H@16 T@24 cw@32 invbase@40 with
     grid_x * block_x = rows * cw threads; rows % 128 == 0, cw % 128 == 0; writes
     T f32 [rows / 128][cw / 128][128][128] (rows % 128 * 128 + d inside a block) =
     the map-decoded 4-bpw mcg weights of each 128-column block times H f32 [128][128],
     summed over c ascending in float32; q, H, T 16-byte and td, inv 4-byte aligned. */
int vybdq_launch_pblock_grid(int kind, uint64_t P, uint32_t grid_x, uint32_t block_x, uint64_t stream);

/* Synchronises the current device, then returns 0 or the error of an invalid parameter block
   launched on it since the previous call (and clears it). */
int vybdq_pblock_status(void);

/* Map-driven EXL3 tile decode, launched as the reference launches exl3deq(q, tab, o) (out_dt
   VYBDQ_F64, exl3.vyb:375-422) and exl3deq32(q, tab, o) (VYBDQ_F32, exl3.vyb:207-242) with grid
   ntiles x 256 (native/host/glm_exl3_check32.vyb:165). tab (8-byte aligned): cw@0, ntiles@8, then
   the 256 x 16-byte map body (4 u16 nibble indices, 4 u8 bit positions, u16 row, u16 col per
   slot). Slot s of tile t: w16 = OR_i nibble(t, nidx_i) << 4 pos_i, y = (w16 * 0xCBAC1FED mod 2^32
   & 0x8FFF8FFF) ^ 0x3B603B60, o[(16 (t / (cw / 16)) + row_s) cw + 16 (t % (cw / 16)) + col_s] =
   fp16(y.lo) + fp16(y.hi) (exact in float32). cw and ntiles are read on the device (the call
   can be captured); a header or map entry out of range (cw % 16, nibble index >= 256, position
   >= 4, row or col >= 16) writes nothing and is reported by the next vybdq_pblock_status(). */
int vybdq_exl3_deq_map(uint64_t q, uint64_t tab, uint64_t out, int out_dt, uint64_t stream);

/* ---- MoE layer ---------------------------------------------------------------------------- */

/* Router alone: idx_out int32 [T, topk] (descending choice, ties to the lower id),
   w_out float32 [T, topk] = sigmoid(logit) renormalised over the selection, times scale.
   bias (float32 [E] or 0) shifts the selection only. Replaces moe_route
   (native/kernels/moe.vyb:28-95); semantics native/glm53/moe_ref.py:68-78. */
int vybdq_moe_route(uint64_t logits, int logits_dt, uint64_t bias, uint64_t idx_out, uint64_t w_out,
                    int64_t T, int64_t E, int64_t topk, double scale, uint64_t stream);

/* Workspace bytes for vybdq_moe_forward, or -1 for an unsupported shape. */
int64_t vybdq_moe_workspace_size(int64_t T, int64_t H, int64_t I, int64_t E, int64_t topk);

/* out [T, H] = sum_s w[t,s] * FFN_{idx[t,s]}(x[t]) + FFN_shared(x[t]) with
   FFN(x) = (silu(min(x Wg, limit)) * clamp(x Wu, -limit, limit)) Wd. Routed weights are GGUF
   expert tensors: w_gate/w_up [E][I rows][H], w_down [E][H rows][I], packed type wtype; the
   shared expert (s_gate/s_up/s_down, or all 0) is one such matrix each. x [T, H] (f32/f16/bf16,
   16-byte aligned), logits [T, E]. Tokens are bucketed per expert on the device and each
   expert's rows run through grouped dequant GEMMs; no host synchronisation. idx_out/w_out
   (optional) receive the routing. Replaces the reference's moe_route/moe_act/moe_down
   (moe.vyb:1-170) for GGUF-quantized experts, with the bucketing and per-expert FFN structure of
   its host loop (native/glm53/glm_engine.vyb:2804-2953); that loop's own weights (EXL3 routed
   experts, a bf16 shared expert) go through vybdq_moe_forward_exl3. */
int vybdq_moe_forward(int wtype, uint64_t x, int x_dt, uint64_t logits, int logits_dt, uint64_t bias,
                      uint64_t w_gate, uint64_t w_up, uint64_t w_down, uint64_t s_gate, uint64_t s_up,
                      uint64_t s_down, uint64_t out, int out_dt, uint64_t idx_out, uint64_t w_out, int64_t T,
                      int64_t H, int64_t I, int64_t E, int64_t topk, double scale, double limit, uint64_t ws,
                      int64_t ws_bytes, uint64_t stream);

/* Largest workspace (bytes) vybdq_moe_forward_noalloc can use: its per-GPU scratch array. At
   H = 6144, I = 2048, E = 256, topk = 8 this covers T <= 233 tokens. */
#define VYBDQ_MOE_NOALLOC_MAX_BYTES (64ll * 1024 * 1024)

/* vybdq_moe_forward without a workspace argument, and without allocating anything: no
   counterpart in the reference; for callers that cannot allocate device memory (code under HIP
   graph capture, tight serving loops, harnesses that forbid hipMalloc). The workspace is a
   library-owned device array of VYBDQ_MOE_NOALLOC_MAX_BYTES per GPU, held until the process
   ends; its address is looked up on the first call on each device (the only set-up step). A
   shape whose vybdq_moe_workspace_size exceeds the array returns VYBDQ_ERR_WORKSPACE before
   any launch. Every call on one GPU shares that GPU's array, so calls that overlap on one GPU
   (several streams or host threads) race: the caller serialises them. Nothing in the array has
   to start at zero (every call rewrites what it reads). Results equal vybdq_moe_forward's. */
int vybdq_moe_forward_noalloc(int wtype, uint64_t x, int x_dt, uint64_t logits, int logits_dt, uint64_t bias,
                              uint64_t w_gate, uint64_t w_up, uint64_t w_down, uint64_t s_gate, uint64_t s_up,
                              uint64_t s_down, uint64_t out, int out_dt, uint64_t idx_out, uint64_t w_out,
                              int64_t T, int64_t H, int64_t I, int64_t E, int64_t topk, double scale,
                              double limit, uint64_t stream);

/* ---- MoE layer with EXL3 routed experts -------------------------------------------------- */

/* Workspace bytes for vybdq_moe_forward_exl3, or -1 for an unsupported shape. */
int64_t vybdq_moe_exl3_workspace_size(int64_t T, int64_t H, int64_t I, int64_t E, int64_t topk);

/* The reference's production GLM-5.3 MoE layer (native/glm53/glm_engine.vyb:2728-2990) in one call:
   out [T, H] = sum_s w[t,s] * FFN_{idx[t,s]}(x[t]) + FFN_shared(x[t]), FFN(x) =
   (silu(min(x Wg, limit)) * clamp(x Wu, -limit, limit)) Wd, routing as vybdq_moe_forward (bias: the
   e_score_correction_bias, selection only). Routed experts are EXL3 4-bpw matrices (mcg codebook):
   `experts` is a device table uint64 [E][9] of the addresses of gate.trellis, gate.suh, gate.svh,
   up.trellis, up.suh, up.svh, down.trellis, down.suh, down.svh of each expert (trellis int16
   [in/16][out/16][64], 16-byte aligned; suh fp16 [in]; svh fp16 [out]; gate/up in = H, out = I;
   down in = I, out = H). The shared expert (s_gate, s_up [I][H], s_down [H][I], bf16 [out][in] as
   mlp.shared_experts.*.weight, 16-byte aligned; or all 0) runs on every token with weight 1.
   x [T, H] f32/f16/bf16 (16-byte aligned), logits [T, E], out F32/F16/BF16; H, I multiples of 128.
   Routing, bucketing, the per-expert EXL3 products (trellis decoded in registers, the Hadamard
   rotations applied to the activations) and the combine all run on the stream: no host loop, no
   host synchronisation, no dequantized weights. Replaces the per-expert loop with exl3_deq32 + f64
   GEMMs (glm_engine.vyb:2804-2953) and the shared expert's deq_bf16 + GEMMs (:2955-2990). */
int vybdq_moe_forward_exl3(uint64_t x, int x_dt, uint64_t logits, int logits_dt, uint64_t bias, uint64_t experts,
                           uint64_t s_gate, uint64_t s_up, uint64_t s_down, uint64_t out, int out_dt,
                           uint64_t idx_out, uint64_t w_out, int64_t T, int64_t H, int64_t I, int64_t E,
                           int64_t topk, double scale, double limit, uint64_t ws, int64_t ws_bytes,
                           uint64_t stream);

/* ---- activation quantizer ------------------------------------------------------------ */

/* xq8 semantics per row and per 32-value block: a = max|x|, d = a/127, q = sat_s8(rne(x*127/a))
   (q = 0, d = 0 for an all-zero block). X: x_dt (F32, F16, BF16) [M, K]; Xq int8 [M, K];
   Xs float32 [M, K/32]. The reference's single-row layout (scales at Y + K) is Xs = Xq + K.
   Replaces xq8 (native/kernels/rgemv7.vyb:195-214). K % 32 == 0. */
int vybdq_quant_q8_act(uint64_t X, uint64_t Xq, uint64_t Xs, int64_t M, int64_t K, int x_dt,
                       uint64_t stream);

#ifdef __cplusplus
}
#endif

#endif /* VYBDQ_H */
