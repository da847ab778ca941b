/*
 * terra_swin.h — C ABI of the MI355X (gfx950) shifted-window attention hot path.
 *
 * The reference (TERRA, pure Python on PyTorch) has no FFI for this path: every
 * step is an ATen call made from Python.  Each entry point below replaces a
 * specific group of those calls; the citation next to each declaration names
 * the reference lines it stands in for (paths relative to the TERRA tree).
 *
 * Conventions
 *   - All tensors are device pointers allocated by the caller (PyTorch).  The
 *     library never allocates or frees device memory on these paths.
 *   - Every entry point validates its arguments on the host before launching
 *     anything and returns TERRA_OK (0) or a negative terra_status.  The text
 *     of the last error of the calling thread is returned by terra_last_error().
 *   - Work is enqueued on `stream` (a hipStream_t passed as void*; NULL is the
 *     default stream).  Nothing synchronises the host.
 *   - Entry points are stateless and reentrant.
 */
#ifndef TERRA_SWIN_H
#define TERRA_SWIN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TERRA_SWIN_ABI_VERSION 1

/* Element types of activations (q/k/v/o, token grids, windows). */
enum terra_dtype {
  TERRA_DTYPE_F32 = 0,
  TERRA_DTYPE_F16 = 1,
  TERRA_DTYPE_BF16 = 2,
  TERRA_DTYPE_U8 = 3 /* partition / reverse only (e.g. per-token land flags) */
};

enum terra_status {
  TERRA_OK = 0,
  TERRA_ERR_NULL = -1,        /* a required pointer is NULL                  */
  TERRA_ERR_DTYPE = -2,       /* dtype not supported by this entry point     */
  TERRA_ERR_SHAPE = -3,       /* inconsistent or out-of-range sizes          */
  TERRA_ERR_ALIGN = -4,       /* pointer / stride not aligned as required    */
  TERRA_ERR_UNSUPPORTED = -5, /* valid request this build does not implement */
  TERRA_ERR_LAUNCH = -6       /* the HIP runtime rejected a launch           */
};

/* Geometry of a token grid and of the window grid cut from it.
 *
 * The window frame is the token grid padded by (pad_top, pad_bottom,
 * pad_left, pad_right) with `pad_value`, then cyclically shifted by
 * (-shift_h, -shift_w) over the padded extents Hp = height+pad_top+pad_bottom,
 * Wp = width+pad_left+pad_right, exactly as torch.roll(x, (-sh, -sw), (1, 2))
 * on the padded tensor.  Hp and Wp must be multiples of `window`.
 *
 * Windows are numbered image-major then row-major over the emitted window rows
 * [win_row_begin, win_row_begin + win_rows) of the Hp/ws x Wp/ws window grid
 * (win_rows <= 0 means all rows).  Windows of an image whose flat index
 * (row-major within the emitted rows) lies outside [valid_begin, valid_end)
 * are pad windows: partition writes them as pad_value and reverse ignores
 * them.  valid_end <= 0 means "all windows valid".
 */
typedef struct terra_swin_geom {
  int32_t batch;    /* B                                   */
  int32_t height;   /* H  (token rows of x / y)            */
  int32_t width;    /* W  (token columns of x / y)         */
  int32_t channels; /* C                                   */
  int32_t window;   /* ws (square windows, N = ws*ws)      */
  int32_t shift_h;  /* 0 <= shift_h < Hp                   */
  int32_t shift_w;  /* 0 <= shift_w < Wp                   */
  int32_t pad_top, pad_bottom, pad_left, pad_right;
  int32_t win_row_begin;
  int32_t win_rows;
  int32_t valid_begin;
  int32_t valid_end;
} terra_swin_geom;

/* Mask modes of terra_swin_attn_fwd. */
enum terra_mask_mode {
  TERRA_MASK_NONE = 0,     /* no additive mask                                  */
  TERRA_MASK_SHIFT = 1,    /* analytic Swin shift mask, from the frame geometry */
  TERRA_MASK_EXPLICIT = 2  /* caller's fp32 [mask_windows, N, N] additive mask  */
};

/* Description of one fused window-attention forward call.
 *
 * q, k, v, o hold `num_windows` windows of `tokens` rows each; row r of window
 * w starts at element (w*tokens + r)*{q,k,v,o}_stride, and head h occupies
 * columns [h*D, (h+1)*D) with D = channels/heads.  Per window w and head h:
 *
 *   S = (q_h k_h^T) * scale + bias_h + M[w]        (fp32)
 *   S[:, j] = pad_key_value   for keys j >= n_real (masked_fill, after M)
 *   o_h = softmax(S) v_h                           (P rounded to the
 *                                                   activation dtype)
 *
 * bias_h[i, j] = bias_table[idx(i, j) * heads + h] with the Swin relative
 * position index idx of a window_h x window_w window; bias_table == NULL
 * disables the bias.  M[w] is the sum of
 *   - the shift mask (mask_mode == TERRA_MASK_SHIFT): mask_value where the
 *     region ids of query and key differ, region ids from the frame
 *     (frame_h x frame_w tokens, shifts shift_h/shift_w, window w at window row
 *     win_row_begin + (w % (win_rows*win_cols)) / win_cols of the frame), or
 *     the caller's explicit_mask[w % mask_windows] (TERRA_MASK_EXPLICIT);
 *   - the land term: mask_value for every key j whose bit j is set in
 *     land_bits[w % mask_windows] (land_bits == NULL disables it).
 *
 * Windows of more than 64 tokens (TERRA's window-32 configuration,
 * configs/model/correctness/credit_hierarchical_swin_correctness_seq.yaml:
 * 21-30, 1024 tokens) run on a tiled online-softmax kernel: bf16, tokens a
 * multiple of 128 up to 4096, D in {64, 128}, n_real == tokens, a positive
 * finite scale, no bias table, mask_mode TERRA_MASK_NONE and no land bits;
 * the rest returns TERRA_ERR_UNSUPPORTED.
 */
typedef struct terra_swin_attn_desc {
  int32_t num_windows; /* B_                                       */
  int32_t tokens;      /* N  (<= 64, or see below)                 */
  int32_t channels;    /* C                                        */
  int32_t heads;       /* nH (D = C / nH in {32, 64, 128})         */
  int32_t window_h, window_w; /* window_h * window_w == tokens     */
  int32_t n_real;      /* keys >= n_real get pad_key_value         */
  int32_t q_stride, k_stride, v_stride, o_stride; /* elements per token row */
  float scale;
  float mask_value;    /* -100.0 in the reference                  */
  float pad_key_value; /* -10000.0 in the reference                */
  int32_t mask_mode;   /* enum terra_mask_mode                     */
  int32_t mask_windows;/* period of explicit_mask / land_bits      */
  int32_t frame_h, frame_w;
  int32_t shift_h, shift_w;
  int32_t win_row_begin, win_rows, win_cols;
} terra_swin_attn_desc;

/* Description of one window-attention backward call: the forward call's
 * descriptor (q/k/v strides, masks, scale; its o_stride is unused) plus the
 * row strides of the output gradient and of the three input gradients. */
typedef struct terra_swin_attn_bwd_desc {
  terra_swin_attn_desc fwd;
  int32_t dout_stride;  /* elements per token row of dout       */
  int32_t dq_stride, dk_stride, dv_stride;
} terra_swin_attn_bwd_desc;

/* Description of one fused Swin attention half-block call.
 *
 * geom: the token grid [B, H, W, C] (channels = C), window (must be 8),
 * shift, frame padding and the emitted window rows / valid-window range,
 * exactly as for terra_swin_partition.  Per emitted window the call computes
 * norm1 -> qkv -> window attention -> proj and adds the result to the window's
 * tokens of x; tokens of windows that are not emitted keep x. */
typedef struct terra_swin_block_desc {
  terra_swin_geom geom;
  int32_t heads;        /* see terra_swin_block_fwd for the shapes      */
  float scale;          /* q k^T scale (head_dim^-0.5 in the reference) */
  float ln_eps;         /* LayerNorm eps                                */
  float mask_value;     /* -100.0 in the reference                      */
  int32_t layernorm;    /* 1: norm1 = LayerNorm(gamma, beta); 0: none   */
  int32_t shift_mask;   /* 1: analytic Swin shift mask over the frame   */
  int32_t land_windows; /* period of land_bits (emitted windows / image) */
  int32_t packed_weights; /* 0: qkv/proj weights in nn.Linear layout;
                             1: in the layout of terra_swin_pack_linear */
} terra_swin_block_desc;

/* Description of one fused MLP half-block call (terra_swin_mlp_fwd). */
typedef struct terra_swin_mlp_desc {
  int32_t tokens;     /* rows of x (any count; B*H*W for a [B, H, W, C] grid) */
  int32_t channels;   /* C: 128, 192, 384 or 768                           */
  int32_t hidden;     /* fc1 out features: 4 * C (mlp_ratio 4)             */
  int32_t layernorm;  /* 1: norm2 = LayerNorm(gamma, beta); 0: none        */
  float ln_eps;       /* LayerNorm eps                                     */
} terra_swin_mlp_desc;

/* ABI version of the loaded library (TERRA_SWIN_ABI_VERSION at build time). */
int terra_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* terra_last_error(void);

/* Fused pad + cyclic shift + window partition.
 * Replaces  torch.roll(x, (-s, -s), dims=(1, 2))      models/transformer.py:179
 *           window_partition(shifted_x, ws)           models/utils.py:35-39
 *           x_windows.view(-1, ws*ws, C)              models/transformer.py:225
 * and the model-level zero padding before the blocks
 *           (models/reference_model/sequential_hierarchical_swin.py:277-278).
 * x: [B, H, W, C] contiguous; windows: [B * nW_emitted, ws*ws, C] contiguous.
 */
int terra_swin_partition(const void* x, void* windows, int dtype,
                         const terra_swin_geom* geom, float pad_value,
                         void* stream);

/* Fused LayerNorm + pad + cyclic shift + window partition.
 * Replaces  x = self.norm1(x)      (nn.LayerNorm over C)  models/transformer.py:98, 150
 * followed by the sequence terra_swin_partition replaces.  Statistics are
 * fp32 over the C channels of each token, y = (x - mean) * rsqrt(var + eps)
 * * gamma + beta, rounded once to the activation dtype (f32 / f16 / bf16).
 * gamma, beta: C floats each, or NULL for 1 / 0.  Padding applies to the
 * normalised grid: frame padding and pad windows are written as pad_value.
 * Needs C * element size to be a multiple of 16 bytes and at most 4096, and
 * C <= 1024.
 */
int terra_swin_partition_ln(const void* x, void* windows, int dtype,
                            const terra_swin_geom* geom, const float* gamma,
                            const float* beta, float eps, float pad_value,
                            void* stream);

/* terra_swin_partition_ln with windows of another dtype than x: fp32 x and
 * bf16 windows (x_dtype == windows_dtype is terra_swin_partition_ln).  Each
 * value is the fp32 LayerNorm output rounded once to bf16 (round to nearest
 * even), bit for bit what terra_swin_partition_ln in fp32 followed by a cast
 * to bf16 gives.  Replaces, in the training step's bf16 autocast region
 * (core/runtime/run_model.py:424-448), norm1 + roll + window_partition
 * (models/transformer.py:150-225) in fp32 and the cast autocast applies to
 * their output at the q/k/v Linear (models/attention.py:244-246), and
 * norm2 (models/mlp.py:159) with the cast at fc1.
 */
int terra_swin_partition_ln_mixed(const void* x, int x_dtype, void* windows, int windows_dtype,
                                  const terra_swin_geom* geom, const float* gamma, const float* beta,
                                  float eps, float pad_value, void* stream);

/* Backward of terra_swin_partition_ln (with pad_value constant: padded slots
 * carry no gradient), plus an optional residual gradient.
 * Replaces the autograd backward of
 *           x = self.norm1(x)      (nn.LayerNorm)        models/transformer.py:98, 150
 *           roll + window_partition                     models/transformer.py:179-225
 * as the training step runs it (core/runtime/run_model.py:362-617), and of
 * norm2 in SequentialMlp (models/mlp.py:159) with an identity frame (window 1,
 * no shift, x viewed as [1, tokens, 1, C]).
 * For every grid token t of x [B, H, W, C]: g = the gradient in dwindows
 * [B * nW_emitted, ws*ws, C] of the slot partition wrote t to (0 where the
 * frame does not emit t or emits a pad window), and
 *   dx[t] = rstd (gamma g - mean_c(gamma g) - xhat mean_c(gamma g xhat))
 *           (+ dresidual[t] if dresidual != NULL)
 * with mean, rstd and xhat = (x - mean) rstd recomputed from x as the forward
 * computes them (fp32), rounded once to the activation dtype.  When dgamma /
 * dbeta are not NULL the call ADDS sum_t g xhat and sum_t g into them (fp32
 * [C]; the caller zeroes them; float atomics, so the summation order varies).
 * gamma: C floats or NULL (1).  dx may equal dresidual but must not overlap x.
 * C <= 1024 in rows of whole 16-byte chunks of at most 4096 bytes.
 */
int terra_swin_partition_ln_bwd(const void* dwindows, const void* x, const void* dresidual, void* dx,
                                int dtype, const terra_swin_geom* geom, const float* gamma, float eps,
                                float* dgamma, float* dbeta, void* stream);

/* terra_swin_partition_ln_bwd with a windows gradient of another dtype than
 * x: a bf16 gradient (of the bf16 windows terra_swin_partition_ln_mixed
 * writes) for fp32 x, dresidual and dx (x_dtype == dwindows_dtype is
 * terra_swin_partition_ln_bwd).  The gradient's bf16 values enter the fp32
 * arithmetic exactly, so the result equals terra_swin_partition_ln_bwd on the
 * gradient cast to fp32 (the backward of autocast's cast).
 */
int terra_swin_partition_ln_bwd_mixed(const void* dwindows, int dwindows_dtype, const void* x,
                                      const void* dresidual, void* dx, int x_dtype,
                                      const terra_swin_geom* geom, const float* gamma, float eps,
                                      float* dgamma, float* dbeta, void* stream);

/* Fused window reverse + inverse cyclic shift + crop (+ residual add).
 * Replaces  window_reverse(attn_windows, ws, H, W)    models/utils.py:41-45
 *           torch.roll(shifted_x, (s, s), dims=(1, 2))  models/transformer.py:246
 *           x = shortcut + x.view(B, H*W, C)          models/transformer.py:296-298
 * y[b, h, w] = residual[b, h, w] (if residual != NULL) + the window token that
 * partition would have read from (b, h, w); tokens whose window is not emitted
 * or is a pad window contribute 0.  y may alias residual.
 */
int terra_swin_reverse(const void* windows, void* y, const void* residual,
                       int dtype, const terra_swin_geom* geom, void* stream);

/* terra_swin_reverse with windows of another dtype than y: bf16 windows into
 * fp32 y and residual (windows_dtype == dtype is terra_swin_reverse).  Each
 * bf16 value is widened exactly and added in fp32, bit for bit what
 * terra_swin_reverse in fp32 on the windows cast to fp32 gives.  Replaces, in
 * the training step's bf16 autocast region (core/runtime/run_model.py:424-448),
 * window_reverse + roll of autocast's bf16 proj output (models/attention.py:281,
 * models/utils.py:41-45, models/transformer.py:246) and the fp32 add
 * x = shortcut + x (models/transformer.py:296-298), which type promotion makes
 * fp32.  Needs C % 4 == 0, 16-byte aligned y / residual and 8-byte aligned
 * windows.  y may alias residual.
 */
int terra_swin_reverse_mixed(const void* windows, int windows_dtype, void* y, const void* residual,
                             int dtype, const terra_swin_geom* geom, void* stream);

/* terra_swin_partition of fp32 x into bf16 windows, each value rounded once
 * (round to nearest even): bit for bit terra_swin_partition in fp32 followed by
 * a cast to bf16.  When column_sums is not NULL the call also ADDS, for each
 * channel, the sum over every window token of the bf16 value written (as
 * fp32; pad slots count pad_value) into column_sums (fp32 [C]; the caller
 * zeroes it; float atomics, so the summation order varies).
 * Replaces, in the training step under bf16 autocast
 * (core/runtime/run_model.py:362-617, 424-448), the autograd backward of
 * window_reverse + roll (models/utils.py:41-45, models/transformer.py:246: a
 * partition of the fp32 grid gradient, pad_value 0), the cast of that gradient
 * to bf16 at the proj Linear's backward and proj's bias gradient
 * grad.sum(0) (models/attention.py:281); with an identity frame (window 1,
 * no shift, x viewed as [1, tokens, 1, C]) the cast of the MLP half's output
 * gradient at fc2's backward and fc2's bias gradient (models/mlp.py:168).
 * Needs C % 4 == 0, C <= 1024, 16-byte aligned x and 8-byte aligned windows.
 */
int terra_swin_partition_mixed(const void* x, int x_dtype, void* windows, int windows_dtype,
                               const terra_swin_geom* geom, float pad_value, float* column_sums,
                               void* stream);

/* Fused per-window multi-head attention core (bf16 or fp32 activations).
 * Replaces  q = q * self.scale                        models/attention.py:256
 *           attn = q @ k.transpose(-2, -1)            models/attention.py:258
 *           relative-position bias gather + add      models/attention.py:260-266
 *           mask add (shift mask buffer)              models/attention.py:269-272
 *           softmax                                   models/attention.py:273-275
 *           (attn @ v).transpose(1, 2).reshape(B_,N,C) models/attention.py:278
 *           padded-key masked_fill(-10000)            models/attention.py:905-907
 * The q/k/v/proj Linear layers stay with the caller.
 */
int terra_swin_attn_fwd(const void* q, const void* k, const void* v, void* o,
                        int dtype, const terra_swin_attn_desc* desc,
                        const float* bias_table, const float* explicit_mask,
                        const uint64_t* land_bits, void* stream);

/* Backward of terra_swin_attn_fwd, for the shapes the forward takes (bf16 or
 * f32, windows up to 8x8 in at most 64 token rows, padded keys, head dim 32,
 * 64 or 128; any mask mode, land bits).  bf16 8x8 windows without padded keys
 * run on an MFMA kernel, the rest on a plain fp32 one.  Windows of more than
 * 64 tokens take the forward's tiled path and its limits (bf16, head dim 64
 * or 128, no bias, mask or padded keys): three passes, the row statistics of
 * the forward (kept in dq until the last pass, so dq must not overlap q, k, v
 * or dout), dk / dv over query tiles, then dq over key tiles.
 * Replaces the autograd backward of the same ATen sequence
 *           models/attention.py:256-278 (matmul, bias gather + add, mask add,
 *           softmax, matmul), as run by the training step
 *           core/runtime/run_model.py:362-617.
 * P is recomputed from q, k and the masks.  Writes
 *   dq = scale * dz k,  dk = scale * dz^T q,  dv = P^T dout     (activation dtype)
 * with dz = P * (dout v^T - rowsum(P * (dout v^T))) per window and head (zero
 * for padded keys, which the forward overwrites with pad_key_value), and,
 * when dbias_table != NULL, ADDS sum over windows of dz[i, j] into
 * dbias_table[idx(i, j) * heads + h] (fp32, same layout as bias_table; the
 * caller zeroes it first; float atomics, so the summation order varies).
 * dq, dk, dv may be column blocks of one [B_, N, 3C] buffer.
 */
int terra_swin_attn_bwd(const void* q, const void* k, const void* v, const void* dout,
                        void* dq, void* dk, void* dv, int dtype,
                        const terra_swin_attn_bwd_desc* desc, const float* bias_table,
                        float* dbias_table, const float* explicit_mask,
                        const uint64_t* land_bits, void* stream);

/* terra_swin_attn_bwd that also ADDS the column sums of the dq, dk and dv it
 * writes (over all windows and tokens, of the bf16 values stored, as fp32)
 * into dq_sums, dk_sums and dv_sums (fp32 [C] each, or NULL; the caller
 * zeroes them; float atomics, so the summation order varies): the bias
 * gradients of the q / k / v Linears (models/attention.py:223-228), which the
 * training step (core/runtime/run_model.py:362-617) otherwise sums from the
 * gradients in a separate pass.  bf16 activations and windows of at most 64
 * tokens (the MFMA tile kernel); other calls return TERRA_ERR_UNSUPPORTED when
 * a sum is requested.
 */
int terra_swin_attn_bwd_sums(const void* q, const void* k, const void* v, const void* dout,
                             void* dq, void* dk, void* dv, int dtype,
                             const terra_swin_attn_bwd_desc* desc, const float* bias_table,
                             float* dbias_table, const float* explicit_mask,
                             const uint64_t* land_bits, float* dq_sums, float* dk_sums,
                             float* dv_sums, void* stream);

/* Fused Swin attention half-block (bf16; 8x8 windows with C = 192 and 6 heads,
 * C = 384 and 12, or C = 768 and 12 heads of dim 64; 7x7 windows with C = 128
 * and 4 heads).
 * Replaces SequentialSwinTransformer.forward   models/transformer.py:142-300:
 *           x = self.norm1(x)                   models/transformer.py:98, 150
 *           roll(-s) + window_partition         models/transformer.py:179-225
 *           qkv = self.qkv(x)                   models/attention.py:244-246
 *           window attention core               models/attention.py:256-278
 *           x = self.proj(x)                    models/attention.py:281
 *           window_reverse + roll(+s)           models/transformer.py:241-246
 *           x = shortcut + x                    models/transformer.py:296-298
 * with the land term of terra_swin_attn_fwd (land_bits[w % land_windows],
 * w = b * emitted windows per image + emitted window index).
 * x, y: [B, H, W, C] bf16 contiguous; y may equal x (in place) but must not
 * overlap it otherwise.  qkv_weight [3C, C] and proj_weight [C, C] bf16
 * (nn.Linear layout); qkv_bias [3C], proj_bias [C], ln_gamma / ln_beta [C]
 * fp32 or NULL; bias_table fp32 [(2 window - 1)^2, heads] or NULL.  Rounding follows the
 * bf16 module: LayerNorm output, q/k/v, P, O and the proj output are rounded
 * to bf16, and the residual add is fp32 rounded once.
 */
int terra_swin_block_fwd(const void* x, void* y, int dtype,
                         const terra_swin_block_desc* desc,
                         const float* ln_gamma, const float* ln_beta,
                         const void* qkv_weight, const float* qkv_bias,
                         const void* proj_weight, const float* proj_bias,
                         const float* bias_table, const uint64_t* land_bits,
                         void* stream);

/* MFMA fragment order of a bf16 [out_features, in_features] weight (out
 * multiple of 16, in multiple of 32) for terra_swin_block_fwd with
 * packed_weights = 1: packed[((rt * in/32 + ks) * 64 + l) * 8 + e] =
 * weight[16 rt + l % 16][32 ks + 8 (l / 16) + e].  A wave then reads each
 * 16 x 32 operand tile as one contiguous 1 KB block.  No reference
 * counterpart: a one-time re-layout of nn.Linear.weight (models/attention.py:
 * 223-228, 281) that the caller keeps with the module.
 */
int terra_swin_pack_linear(const void* weight, void* packed, int dtype,
                           int out_features, int in_features, void* stream);

/* Fused MLP half-block (bf16 activations).
 * Replaces SequentialMlp.forward              models/mlp.py:152-172:
 *           x = self.norm2(x)                  models/mlp.py:159 (nn.LayerNorm)
 *           x = self.fc1(x)                    models/mlp.py:162 (C -> 4C)
 *           x = self.act(x)                    models/mlp.py:165 (nn.GELU, erf form)
 *           x = self.fc2(x)                    models/mlp.py:168 (4C -> C)
 *           x = shortcut + x                   models/mlp.py:171
 * per token row of x [tokens, C] (bf16, contiguous).  y may equal x (in
 * place) but must not overlap it otherwise.  fc1_weight / fc2_weight are the
 * bf16 nn.Linear weights [4C, C] / [C, 4C] in the layout of
 * terra_swin_pack_linear; fc1_bias [4C], fc2_bias [C], ln_gamma / ln_beta
 * [C] fp32 or NULL.  Rounding follows the bf16 module: LayerNorm output,
 * fc1 output (bias added in fp32), GELU output and fc2 output are rounded to
 * bf16, and the residual add is fp32 rounded once.
 */
int terra_swin_mlp_fwd(const void* x, void* y, int dtype,
                       const terra_swin_mlp_desc* desc,
                       const float* ln_gamma, const float* ln_beta,
                       const void* fc1_weight, const float* fc1_bias,
                       const void* fc2_weight, const float* fc2_bias,
                       void* stream);

/* Epilogues of terra_swin_linear. */
enum terra_linear_epilogue {
  TERRA_LINEAR_STORE = 0, /* y = bf16(x W^T + b)                            */
  TERRA_LINEAR_GELU = 1   /* y = GELU(bf16(x W^T + b)), nn.GELU (erf form)   */
};

/* Token-row linear layer (bf16, fp32 accumulation) with a fused epilogue:
 *   y[m] = epilogue(x[m] W^T + b)        for rows m < rows
 * x [rows, in_features] with row stride x_stride elements (a multiple of 8),
 * y [rows, out_features] with row stride y_stride (a multiple of 4); W the
 * bf16 nn.Linear weight [out_features, in_features] in the layout of
 * terra_swin_pack_linear; bias fp32 [out_features] or NULL.  in_features a
 * multiple of 64, out_features a multiple of 256 up to 4096; x_stride * 512
 * bytes under 4 GiB.  y must not overlap x.
 * Rounding: the sum plus bias is rounded once to bf16; TERRA_LINEAR_GELU then
 * applies nn.GELU to that bf16 value in fp32 and rounds to bf16.
 * Replaces  self.fc1(x); self.act(x)        models/mlp.py:162-165
 *           (nn.Linear, nn.GELU())          models/mlp.py:138-150
 * and, with TERRA_LINEAR_STORE, any nn.Linear over token rows
 *           (q/k/v models/attention.py:223-228, 244-246).
 */
int terra_swin_linear(const void* x, void* y, int dtype, int64_t rows,
                      int in_features, int out_features,
                      int64_t x_stride, int64_t y_stride,
                      const void* weight_packed, const float* bias,
                      int epilogue, void* stream);

/* Linear layer plus residual add (bf16), optionally scattering the rows from
 * window order back to the token grid:
 *   y[t(m)] = bf16(residual[t(m)] + bf16(x[m] W^T + b))
 * x [rows, in_features] contiguous; W, bias as for terra_swin_linear.
 * geom NULL: t(m) = m; residual and y are [rows, out_features].
 *   Replaces  x = self.fc2(x); x = shortcut + x      models/mlp.py:168-171
 * geom non-NULL (8x8 windows, every frame window emitted: no window-row or
 * valid-window range): x holds the window tokens [B * nW, 64, C] in the order
 * of terra_swin_partition, rows = B * nW * 64, out_features = C; residual and
 * y are [B, H, W, C] and t(m) is the grid token the partition read row m
 * from (frame-padding rows are dropped).
 *   Replaces  x = self.proj(x)                       models/attention.py:281
 *             window_reverse(attn_windows, ws, H, W) models/utils.py:41-45
 *             torch.roll(x, (s, s), (1, 2))          models/transformer.py:246
 *             x = shortcut + x                       models/transformer.py:296-298
 * y may equal residual but must not overlap it otherwise, nor overlap x.
 */
int terra_swin_linear_residual(const void* x, const void* residual, void* y,
                               int dtype, int64_t rows,
                               int in_features, int out_features,
                               const void* weight_packed, const float* bias,
                               const terra_swin_geom* geom, void* stream);

/* Backward of the MLP half's activation in the training step
 * (core/runtime/run_model.py:362-617): for rows x features tensors
 *   dh = dout * (Phi(h) + h phi(h)),
 *   Phi(h) = 0.5 (1 + erf(h / sqrt 2)),  phi(h) = exp(-h^2 / 2) / sqrt(2 pi),
 * computed in fp32 and rounded once to dtype (bf16 or f32), i.e. the autograd
 * backward of x = self.act(x) (nn.GELU, erf form, models/mlp.py:165) with h =
 * fc1's output.  When column_sums is not NULL the call also ADDS each column's
 * sum of the dh values written (as fp32) into column_sums (fp32 [features];
 * the caller zeroes it; float atomics, so the summation order varies): fc1's
 * bias gradient grad.sum(0) (models/mlp.py:162).  Needs features * element
 * size to be a multiple of 16 bytes and at most 8192, 16-byte aligned
 * tensors, and dh not overlapping dout or h.
 */
int terra_swin_gelu_bwd(const void* dout, const void* h, void* dh, int dtype, int64_t rows,
                        int features, float* column_sums, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TERRA_SWIN_H */
