/*
 * flicker_hip.h -- C ABI of libflicker_hip.so, the MI355X (gfx950) kernels behind
 * flicker_amd's drop-in replacements for kelechi-c/flicker's DiT attention hot path.
 *
 * Conventions for every entry point:
 *   - The caller owns every buffer (device memory).  The library allocates nothing and
 *     never synchronises the host.  Two pieces of state outlive a call:
 *       * flk_attend_split_static_to's fixed scratch buffer, a file-scope device array of
 *         FLK_ATTEND_STATIC_SCRATCH_BYTES per GPU (reserved on a GPU when the library's
 *         attend code object is loaded there, i.e. for every attend user), and the device
 *         address of it that the first such call on a GPU looks up and caches;
 *       * the int counters in a flk_attend_balanced_to workspace (the caller's memory): each
 *         call leaves them tagged with its own epoch, a process-wide call number the library
 *         keeps, and no later call needs them reset.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the default stream).
 *   - bf16 tensors are passed as `void*` to raw 16-bit bf16 storage.
 *   - Return value: FLK_OK (0) on success, a negative FLK_E_* code for an argument
 *     the kernel cannot take (checked before anything is launched), or a positive
 *     hipError_t if the launch itself failed.  flk_status_string() names each code.
 *   - Lengths, token and channel counts are `int`; one within a tile (at most 256) of
 *     INT32_MAX is FLK_E_INVALID, since the kernels index whole tiles in 32 bits.
 */
#ifndef FLICKER_HIP_H
#define FLICKER_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FLK_OK 0
#define FLK_E_INVALID (-1)     /* a size, count or offset out of range          */
#define FLK_E_ALIGN (-2)       /* a pointer or stride breaks the 16-byte rule    */
#define FLK_E_UNSUPPORTED (-3) /* a shape the library has no kernel for        */
#define FLK_E_SCRATCH (-4)     /* needs more than a fixed scratch buffer holds  */

/* ABI revision of this header (bumped on any signature change). */
int flk_abi_version(void);

/* Static, human-readable text for a return code of any entry point. */
const char* flk_status_string(int status);

/*
 * Fused head transpose + QK-RMSNorm + multi-axis RoPE.
 * Replaces kernels.qk_prep (src/flicker/kernels.py:57-91; tile body _body :35-53).
 *   qkv        (batch, length, 3*num_heads*head_dim) bf16; element (b, t, c) lives at
 *              qkv + b*qkv_batch_stride + t*qkv_row_stride + c (strides in elements,
 *              multiples of 8; the last axis contiguous)
 *   cos, sin   (length, head_dim) float32 lane tables (kernels.lane_pair layout), row t at
 *              t*table_row_stride floats (multiple of 4)
 *   q_scale, k_scale (head_dim,) bf16 (scale_is_f32 = 0) or float32 (scale_is_f32 = 1)
 *   q_gain     multiplies the rotated query before its bf16 rounding (1.0 = none)
 *   q_out, k_out, v_out  (batch, num_heads, out_length, head_dim) bf16; token t of this call
 *              is written at sequence index out_offset + t (out_offset + length <= out_length),
 *              so two calls can fill one concatenated text|image buffer
 * head_dim must be 128.
 */
int flk_qk_prep(const void* qkv, int64_t qkv_batch_stride, int64_t qkv_row_stride,
                const float* cos, const float* sin, int64_t table_row_stride,
                const void* q_scale, const void* k_scale, int scale_is_f32, float q_gain,
                int batch, int length, int num_heads, int head_dim,
                void* q_out, void* k_out, void* v_out, int64_t out_length, int64_t out_offset,
                void* stream);

/*
 * The plain branch of qkv_prep with float32 norm scales (src/flicker/modules.py:78-80: heads,
 * qk_norm, apply_rope).  There rms_norm's bf16(x * rsqrt) * scale promotes to float32
 * (src/flicker/nn.py:27) and apply_rope casts its float32 rotation back to that dtype
 * (src/flicker/rope.py:28), so q and k come out float32: the rotation of the float32 product,
 * with no rounding after it and no query gain.  v is the bf16 copy, as in flk_qk_prep.
 *   q_scale, k_scale (head_dim,) float32
 *   cos, sin   lane tables of the plain branch's rope table at gain 1 (kernels.lane_pair layout)
 *   q_out, k_out (batch, num_heads, out_length, head_dim) float32; v_out bf16 of that shape
 * Every other argument as flk_qk_prep.  With bf16 scales the plain branch's q and k are
 * bf16 and flk_qk_prep at q_gain 1 computes them.
 */
int flk_qk_prep_f32(const void* qkv, int64_t qkv_batch_stride, int64_t qkv_row_stride,
                    const float* cos, const float* sin, int64_t table_row_stride,
                    const float* q_scale, const float* k_scale, int batch, int length,
                    int num_heads, int head_dim, float* q_out, float* k_out, void* v_out,
                    int64_t out_length, int64_t out_offset, void* stream);

/*
 * flk_qk_prep with the RoPE lanes computed in the kernel from position ids instead of read
 * from cos / sin tables: the fused form of qk_prep(qkv, ..., lane_pair(embed_nd(ids))),
 * i.e. kernels.qk_prep (src/flicker/kernels.py:57-91) over rope.embed_nd
 * (src/flicker/rope.py:9-21) and kernels.lane_pair (kernels.py:28-31).  The cos / sin values
 * are bit-identical to those flk_rope_lanes stores, so the outputs equal flk_qk_prep's with
 * those tables; the two (length, head_dim) f32 tables are neither built nor read.
 *   ids        (length, n_axes) float32 positions, row t at t*ids_row_stride floats; shared
 *              by every batch element (lane_pair takes batch 0)
 *   n_axes, axes_dim, theta  as flk_rope_lanes; sum(axes_dim) must equal head_dim
 * Every other argument as flk_qk_prep.
 */
int flk_qk_prep_ids(const void* qkv, int64_t qkv_batch_stride, int64_t qkv_row_stride,
                    const float* ids, int64_t ids_row_stride, int n_axes, const int* axes_dim,
                    float theta, const void* q_scale, const void* k_scale, int scale_is_f32,
                    float q_gain, int batch, int length, int num_heads, int head_dim,
                    void* q_out, void* k_out, void* v_out, int64_t out_length,
                    int64_t out_offset, void* stream);

/*
 * Bounded flash attention: softmax without the running max, legal because the
 * QK-norm scales bound every logit (checked at load time, kernels.logit_bound).
 * Replaces kernels.attend (src/flicker/kernels.py:105-145).
 *   q, k, v, o (batch, heads, length, head_dim) bf16, contiguous; q is already scaled by
 *   1/sqrt(head_dim).  o = bf16(sum_j bf16(exp(q.k_j)) v_j / sum_j f32(bf16(exp(q.k_j)))).
 * Any length >= 1 (tail tiles are masked).  head_dim must be 128.  How queries are tiled
 * (flk_attend_kernel) does not change the result.
 */
int flk_attend(const void* q, const void* k, const void* v, void* o,
               int batch, int heads, int length, int head_dim, void* stream);

/*
 * Name of the kernel flk_attend / flk_attend_to launch for this shape (no counterpart in the
 * reference; for profilers and benchmarks, which match kernel traces by name):
 * "attend_kernel" (one block per 256-query tile), "attend_tile192_kernel" (192-query tiles:
 * grids that fit the 256 CUs in one round either way) or "attend_rounds_kernel" (whole
 * rounds of 256-query tiles per XCD, the tiles left over re-tiled by 192 queries); "" for an
 * empty shape.  The three give the same output bits.
 */
const char* flk_attend_kernel(int batch, int heads, int length);

/*
 * flk_attend writing O through strides (elements): o[b, h, t, :] starts at
 * o + b*o_batch_stride + h*o_head_stride + t*o_row_stride, the head_dim values contiguous.
 * With (L*H*D, D, H*D) this is the token-major (batch, length, heads*head_dim) layout that
 * merge_heads produces (src/flicker/modules.py:63-65), so attention writes the merged output
 * directly instead of a (B, H, L, D) tensor plus a transposing copy (modules.py:157,198).
 * Strides must be multiples of 4 elements, o 8-byte aligned, o_row_stride >= head_dim.
 */
int flk_attend_to(const void* q, const void* k, const void* v, void* o,
                  int batch, int heads, int length, int head_dim,
                  int64_t o_batch_stride, int64_t o_head_stride, int64_t o_row_stride, void* stream);

/*
 * flk_attend_to for grids too small to fill the GPU (few heads: one GPU's share of a
 * head-parallel run, or short sequences).  It computes the same attend (src/flicker/
 * kernels.py:105-145), with the keys cut into `splits` ranges of equal length (in 64-key
 * tiles, +-1 tile).
 * Each (b, h, 256-query tile, range) block sums its own acc and l.  A second kernel adds the
 * ranges in order, as plain sums: the reference keeps no running max, so no rescaling is
 * needed.  It then writes o = bf16(acc / l).
 *
 * Only the f32 summation order differs from flk_attend_to.  Results are deterministic for
 * a given (batch, heads, length, splits).
 *
 * Arguments:
 * - 1 <= splits <= ceil(length / 256); splits == 1 is flk_attend_to itself.
 * - `workspace`: caller-owned, 16-byte aligned scratch of at least
 *   splits * batch * heads * ceil(length / 256) * 512 * 65 * 4 bytes (f32 partial acc
 *   and l of every 256-query tile).  Nothing in it needs to be initialised; it is dead
 *   after the call.
 * - Other arguments as flk_attend_to.
 */
int flk_attend_split_to(const void* q, const void* k, const void* v, void* o,
                        int batch, int heads, int length, int head_dim,
                        int64_t o_batch_stride, int64_t o_head_stride, int64_t o_row_stride,
                        int splits, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * flk_attend_split_to without a caller workspace: it allocates nothing (no hipMalloc, no
 * allocating library call).  No counterpart in the reference; it is for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid it).
 * The partials live in a fixed device buffer of FLK_ATTEND_STATIC_SCRATCH_BYTES per GPU, a
 * file-scope __device__ array of the attend code object: it is reserved on a GPU as soon as
 * the library's attend kernels are loaded there (every attend user holds it, whether or not
 * it calls this function) and kept until the process ends.  It is enough for every split that
 * flk_attend_plan picks (at most 256 (b, h, 256-query tile, range) blocks of 133120 bytes).
 *   - A call whose workspace (as flk_attend_split_to's) would exceed the buffer returns
 *     FLK_E_SCRATCH before anything is launched; splits == 1 needs no buffer.
 *   - Every call on one GPU shares that GPU's buffer: calls that overlap on one GPU (on
 *     different streams, or from different threads) race and must be ordered by the caller.
 *     Nothing in the buffer has to start at zero.
 *   - The first call on a GPU looks up the buffer's device address with that GPU current
 *     (the GPU of `stream`, or the current one for the NULL stream).
 * Other arguments and results as flk_attend_split_to, bit for bit.
 */
#define FLK_ATTEND_STATIC_SCRATCH_BYTES 34078720
int flk_attend_split_static_to(const void* q, const void* k, const void* v, void* o,
                               int batch, int heads, int length, int head_dim,
                               int64_t o_batch_stride, int64_t o_head_stride, int64_t o_row_stride,
                               int splits, void* stream);

/*
 * flk_attend_to with the work spread evenly over the GPU's 256 CUs.  The same attend
 * (src/flicker/kernels.py:105-145): instead of one block per (b, h, 256-query tile) -- 432
 * tiles at the Klein 1024^2 shape, 1.69 rounds of 256 CUs -- 256 persistent blocks, 32 per
 * XCD.  Each XCD takes a contiguous range of tiles; its CUs do whole tiles for as many full
 * rounds as the range holds, and the key tiles of the tiles left over are laid end to end
 * and cut into 32 equal ranges, one per CU, so a leftover tile may be shared by a few CUs.
 * The pieces' (acc, l) partials are summed by whichever piece finishes last, always in the
 * same order (plain sums: the reference keeps no running max); no block waits for another.
 * Only the f32 summation order of the shared tiles differs from flk_attend_to; the results
 * are deterministic for a given shape.
 *   - Takes every shape flk_attend_to takes; flk_attend_balanced_plan says whether it is the
 *     faster launch for a shape.
 *   - `workspace`: caller-owned, 16-byte aligned, at least flk_attend_balanced_plan's bytes.
 *     The int counters at its counters_offset hold (epoch << 8) | arrivals, the epoch a tag
 *     of each call (1 .. 2^24 - 1 in turn); a count from another epoch or an already complete
 *     count is read as no arrivals, so the counters are never reset.  Allocate them zeroed
 *     (epoch 0 is never issued); after that any state an earlier call left -- even two calls
 *     that overlapped on the workspace, whose own results are then undefined -- is valid
 *     for the next call that has the workspace to itself.  Calls that share one workspace
 *     must not overlap (one workspace per stream).
 *   - Other arguments as flk_attend_to.
 */
int flk_attend_balanced_to(const void* q, const void* k, const void* v, void* o,
                           int batch, int heads, int length, int head_dim,
                           int64_t o_batch_stride, int64_t o_head_stride, int64_t o_row_stride,
                           void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Whether flk_attend_balanced_to is the faster launch for a shape (*grid = its block count,
 * 256, else 0: with fewer than 256 tiles, or a last round of tiles filling more than 5/8 of
 * the CUs, one block per tile -- or the key split -- is as fast or faster), its workspace
 * size and the byte offset of its hand-off counters, to be allocated zeroed (both independent
 * of the shape).  No device work.
 */
int flk_attend_balanced_plan(int batch, int heads, int length, int* grid, int64_t* workspace_bytes,
                             int64_t* counters_offset);

/*
 * The split count flk_attend_split_to should use for a shape, and its workspace size.
 * *splits = 1 (workspace 0) when the plain grid already has >= 192 blocks of 256 queries.
 * Otherwise it takes as many ranges as fill the 256 CUs once, keeping at least 512 keys per
 * range.  A pure function of its arguments; no device work.
 */
int flk_attend_plan(int batch, int heads, int length, int* splits, int64_t* workspace_bytes);

/*
 * RoPE angle tables.  Replaces rope.embed_nd / rope.rope_freqs (src/flicker/rope.py:9-21):
 *   ids  (length, n_axes) float32 positions, row t at t*ids_row_stride floats
 *   axes_dim  host array of n_axes even ints (1 <= n_axes <= 8)
 *   pe   (length, P, 2, 2) float32 with P = sum(axes_dim)/2: [[cos, -sin], [sin, cos]] of
 *        angle = id * theta^(-2k/dim) for pair k of each axis, axes concatenated in order.
 */
int flk_rope_embed(const float* ids, int64_t ids_row_stride, int64_t length, int n_axes,
                   const int* axes_dim, float theta, float* pe, void* stream);

/*
 * Lane tables from a pe table.  Replaces kernels.lane_pair (src/flicker/kernels.py:28-31):
 *   pe (length, pairs, 2, 2) float32 -> cos, sin (length, 2*pairs) float32 with
 *   cos[t,2j] = cos[t,2j+1] = pe[t,j,0,0], sin[t,2j] = -pe[t,j,1,0], sin[t,2j+1] = pe[t,j,1,0].
 */
int flk_lane_pair(const float* pe, int64_t length, int pairs, float* cos, float* sin, void* stream);

/*
 * flk_rope_embed followed by flk_lane_pair in one pass (no pe table in memory).
 * Produces the same cos/sin tables as kernels.lane_pair(rope.embed_nd(ids)).
 */
int flk_rope_lanes(const float* ids, int64_t ids_row_stride, int64_t length, int n_axes,
                   const int* axes_dim, float theta, float* cos, float* sin, void* stream);

/* ---- int8 SmoothQuant W8A8 QKV projection ------------------------------------------
 * Replaces the bf16 projection `linear(x, w) = x @ w` (src/flicker/nn.py:13-14) where the
 * reference calls it for the fused QKV projection (src/flicker/modules.py:128,132,186:
 * img/txt qkv of double blocks, linear1 of single blocks).  The reference has no
 * quantisation; the replacement is defined by this formula, reproduced bit for bit
 * (single IEEE f32 operations, round-to-nearest-even, correctly rounded / and sqrt):
 *   s_j  = sqrt(max_t|X[t,j]|) / sqrt(max_o|W[j,o]|)   (1 if either is 0), inv_s_j = 1/s_j
 *   w_o  = max_j|f32(W[j,o])*s_j| / 127 (1 if 0);  Wq = clamp(rint(f32(W)*s_j / w_o), +-127)
 *   a_t  = max_j|f32(X[t,j])*inv_s_j| / 127 (1 if 0);  Xq = clamp(rint(f32(X)*inv_s_j / a_t), +-127)
 *   acc  = Xq . Wq (int32, exact);  Y = bf16((f32(acc) * a_t) * w_o)
 * bf16 matrices are row-major with a row stride in elements. */

/* Calibration: out[r] = max_c |x[r,c]| of a bf16 (rows, cols) matrix (cols % 8 == 0). */
int flk_absmax_rows(const void* x, int64_t rows, int64_t cols, int64_t row_stride, float* out,
                    void* stream);

/* Calibration: out[c] = max_r |x[r,c]|; with accumulate != 0, max(out[c], ...) so the
 * activation statistics of several calibration batches can be folded in. */
int flk_absmax_cols(const void* x, int64_t rows, int64_t cols, int64_t row_stride, int accumulate,
                    float* out, void* stream);

/* s and inv_s (k,) f32 from the activation and weight channel maxima. */
int flk_smooth_factors(const float* x_absmax, const float* w_absmax, int64_t k, float* s,
                       float* inv_s, void* stream);

/* Weight W (k, n) bf16 (the reference's (in, out) layout) -> wq_t (n, k) int8, stored
 * transposed so GEMM operands are k-contiguous, and w_scale (n,) f32.  k % 64 == 0,
 * n % 8 == 0. */
int flk_quantize_weight(const void* w, int64_t w_row_stride, const float* s, int k, int n,
                        int8_t* wq_t, float* w_scale, void* stream);

/* Activation X (m, k) bf16 -> xq (m, k) int8 and a_scale (m,) f32 (per token).
 * k % 8 == 0, k <= 8192. */
int flk_quantize_act(const void* x, int64_t x_row_stride, const float* inv_s, int m, int k,
                     int8_t* xq, float* a_scale, void* stream);

/* flk_quantize_act of the modulated block input: X = modulate(x) (src/flicker/modules.py:38-40,
 * norm=True: (1 + scale) * layer_norm(x) + shift, each bf16 operation rounded; layer_norm per
 * src/flicker/nn.py:17-21 with its mean and variance summed in float64 and rounded to float32
 * once) is computed from the raw x and quantised in the same pass.  Replaces the reference's
 * modulate(...) feeding linear(., qkv.weight) (modules.py:128,132,186).
 *   x (m, k) bf16 (row stride in elements); token row r belongs to batch entry
 *   r / tokens_per_batch, whose modulation rows are shift / scale + entry * mod_batch_stride
 *   (k bf16 values each).  x_mod (optional, NULL to skip) receives X as bf16 (m, k).
 * k % 8 == 0, k <= 8192; strides multiples of 8; shift, scale, x_mod 16-byte aligned. */
int flk_quantize_act_modulated(const void* x, int64_t x_row_stride, const void* shift, const void* scale,
                               int64_t mod_batch_stride, int tokens_per_batch, const float* inv_s, int m, int k,
                               int8_t* xq, float* a_scale, void* x_mod, int64_t x_mod_row_stride, void* stream);

/* Two flk_quantize_act_modulated activations of the same width k in one launch: a double
 * block's text and image inputs, each with its own modulation rows and smoothing factors
 * (modules.py:38-40 for img_mod and txt_mod, feeding the two projections of modules.py:
 * 127-135).  The 512 text rows would otherwise be a small launch of their own.  Per stream
 * the arguments and results are exactly flk_quantize_act_modulated's; an empty stream
 * (m_i == 0) is skipped. */
int flk_quantize_act_modulated_pair(const void* x0, int64_t x_row_stride0, const void* shift0, const void* scale0,
                                    int64_t mod_batch_stride0, int tokens_per_batch0, const float* inv_s0, int m0,
                                    int8_t* xq0, float* a_scale0, void* x_mod0, int64_t x_mod_row_stride0,
                                    const void* x1, int64_t x_row_stride1, const void* shift1, const void* scale1,
                                    int64_t mod_batch_stride1, int tokens_per_batch1, const float* inv_s1, int m1,
                                    int8_t* xq1, float* a_scale1, void* x_mod1, int64_t x_mod_row_stride1, int k,
                                    void* stream);

/* y (m, n) bf16 = rescaled int8 product of xq (m, k) and wq_t (n, k); when acc_or_null is
 * given, the exact int32 products are also written there as (m, n).  k % 128 == 0,
 * n % 4 == 0, y 8-byte aligned with y_row_stride % 4 == 0. */
int flk_w8a8_gemm(const int8_t* xq, const int8_t* wq_t, const float* a_scale, const float* w_scale,
                  int m, int k, int n, void* y, int64_t y_row_stride, int32_t* acc_or_null,
                  void* stream);

/* int8 projection and qk_prep in one kernel: qk_prep(bf16(rescaled xq . wq_t^T)) with the
 * GEMM's epilogue doing the RMSNorm + RoPE of each finished head row, so the projected
 * activation Y never goes to memory.  Replaces the pair linear(x, w) (src/flicker/nn.py:13-14
 * at modules.py:128,132,186) -> qk_prep (src/flicker/kernels.py:57-91), with the int8
 * projection above; bit-identical to flk_w8a8_gemm followed by flk_qk_prep.
 *   xq (batch*length, k) int8, wq_t (3*num_heads*head_dim, k) int8, a_scale / w_scale as for
 *   flk_w8a8_gemm; cos, sin, q_scale, k_scale, scale_is_f32, q_gain, q_out/k_out/v_out,
 *   out_length and out_offset as for flk_qk_prep (output row m = b*length + t).
 * k % 128 == 0, head_dim must be 128. */
int flk_w8a8_qk_prep(const int8_t* xq, const int8_t* wq_t, const float* a_scale, const float* w_scale, int k,
                     const float* cos, const float* sin, int64_t table_row_stride,
                     const void* q_scale, const void* k_scale, int scale_is_f32, float q_gain,
                     int batch, int length, int num_heads, int head_dim,
                     void* q_out, void* k_out, void* v_out, int64_t out_length, int64_t out_offset,
                     void* stream);

/* Two flk_w8a8_qk_prep projections in one launch, writing into the same q/k/v buffers:
 * a double block's text and image streams.  Replaces the two linear + qk_prep pairs of
 * modules.py:127-135 (txt_attn.qkv and img_attn.qkv, each with its own norm scales and RoPE
 * rows) followed by the concatenations of modules.py:136-139.  The small text projection
 * (512 tokens, 72 tiles) runs on the CUs the image projection leaves idle in its last
 * round, instead of taking a launch of its own.
 *
 * Per stream i: xq_i (batch*length_i, k), wq_t_i, a_scale_i, w_scale_i, cos_i/sin_i (length_i
 * rows), q_scale_i/k_scale_i, and the sequence offset out_offset_i at which its tokens go.
 * Shared: k, table_row_stride, scale_is_f32, q_gain, batch, num_heads, head_dim, the
 * outputs and out_length.
 *
 * Each stream gets exactly flk_w8a8_qk_prep's result (bit-identical); an empty stream
 * (length_i == 0) is skipped. */
int flk_w8a8_qk_prep_pair(const int8_t* xq0, const int8_t* wq_t0, const float* a_scale0, const float* w_scale0,
                          const float* cos0, const float* sin0, const void* q_scale0, const void* k_scale0,
                          int length0, int64_t out_offset0,
                          const int8_t* xq1, const int8_t* wq_t1, const float* a_scale1, const float* w_scale1,
                          const float* cos1, const float* sin1, const void* q_scale1, const void* k_scale1,
                          int length1, int64_t out_offset1,
                          int k, int64_t table_row_stride, int scale_is_f32, float q_gain, int batch,
                          int num_heads, int head_dim, void* q_out, void* k_out, void* v_out,
                          int64_t out_length, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLICKER_HIP_H */
