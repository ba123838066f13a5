/*
 * CPU restatement of wavo's CPU backend (the parity oracle).
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load or call anything here, and only as the checker or the timed CPU baseline.  The product
 * (wavo_amd/, libwavo_hip.so) never links or calls it.
 *
 * It follows the *portable* arithmetic of the reference's CPU backend (src/cpu/): GEMM operands
 * rounded to f16 (`to_half`), f32 fused multiply-adds summed over k in order, Cephes exp, A&S GELU,
 * 8-lane row sums.  Each function cites the reference file:line it restates.  Activations are f32
 * row-major [rows][cols] throughout, as in the reference.
 *
 * Parity pins (see tests/test_oracle.py): every function is checked against the reference's
 * unit-test known answers (src/gguf.rs, src/cpu/gemm.rs, src/gpu/mod.rs test recipes), closed forms
 * or brute force.  Q4_0 has no reference implementation (ggml type 2 is absent from src/gguf.rs);
 * it is pinned by the ggml block definition and brute force only.
 */
#ifndef WAVO_ORACLE_H
#define WAVO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (src/gguf.rs:22-30; Q4_0 = 2 from ggml's enum). */
enum { OX_F32 = 0, OX_F16 = 1, OX_Q4_0 = 2, OX_Q8_0 = 8 };

/* Epilogue modes, equal to Epilogue::params (src/gpu/mod.rs:445-455). */
enum { OX_BIAS = 0, OX_SILU = 1, OX_RELU = 2, OX_RESIDUAL = 3, OX_GELU = 4, OX_GELU_RESIDUAL = 5,
       OX_TANH = 6 };

/* --- scalars --------------------------------------------------------------------------------- */
float ox_to_half(float x);          /* src/cpu/gemm.rs:213-221 */
float ox_half_to_float(uint16_t h); /* IEEE binary16 -> f32 (the `half` crate's to_f32) */
uint16_t ox_float_to_half_bits(float x); /* IEEE RNE, overflow to inf (half::f16::from_f32) */
float ox_exp(float x);              /* src/cpu/ops.rs:16-26 (Cephes expf) */
float ox_silu(float x);             /* src/cpu/ops.rs:28-31 */
float ox_gelu(float x);             /* src/cpu/ops.rs:33-40 */
float ox_dot(const float *a, const float *b, size_t n); /* src/cpu/mod.rs:20-43 */

/* --- weights --------------------------------------------------------------------------------- */
/* Bytes of `n` weights of ggml type `type` (src/gguf.rs:32-38, + Q4_0 18 B / 32). */
size_t ox_type_size(int type, size_t n);
/* Dequantize `n` weights of `type` (src/gguf.rs:274-287 Tensor::to_f32; Q4_0 per ggml). */
int ox_dequant(int type, const void *src, float *dst, size_t n);
/* ggml quantize_row_q8_0_ref / q4_0_ref, the quantizers of scripts/convert.py:198-209. */
void ox_quantize_q8_0(const float *x, void *dst, size_t n);
void ox_quantize_q4_0(const float *x, void *dst, size_t n);

/* A linear layer y = x·Wᵀ + b with W [n][k] kept in its GGUF bytes (src/cpu/gemm.rs:35-122). */
typedef struct ox_linear {
  int n, k, type;
  uint8_t *w;   /* n rows of k weights, GGUF bytes, rows contiguous */
  float *bias;  /* n values (zeros without a bias) */
} ox_linear;

/* Stack `count` weights (each rows_i x k of one type, GGUF bytes) along n, with `bias` of n values
 * or NULL (src/cpu/gemm.rs:45-72).  Returns NULL on a shape/type error. */
ox_linear *ox_linear_new(int type, int k, int count, const void *const *ws, const int *rows,
                         const float *bias);
void ox_linear_free(ox_linear *l);
/* Row r of W in f32, dequantized, not rounded (src/cpu/gemm.rs:75-82). */
void ox_linear_row(const ox_linear *l, int r, float *out);

/* c[m][n] = epi(h(a)·h(W)ᵀ + b), h = to_half, f32 FMA over k in order (src/cpu/gemm.rs:126-177,
 * portable path :163-176; jobs :228-269; finish :339-352). */
void ox_gemm(const float *a, const ox_linear *l, float *c, int m, int epi, float alpha);
/* The same with the GPU Linear's output layout (src/gpu/mod.rs:752-834 upload_linear and the
 * reference's GEMM test :1878-1945): rows of c are `cols + dual` wide, `cols` = n if n % 32 == 0
 * else n rounded up to 64; columns n..cols get epi(0); `dual` more biases in `bias2` write the
 * first `dual` outputs again at cols.. without an epilogue. */
void ox_gemm_wide(const float *a, const ox_linear *l, float *c, int m, int epi, float alpha,
                  const float *bias2, int dual);
/* c[n] = epi(x·Wᵀ + b), W not rounded, dot() per row (src/cpu/gemm.rs:181-208). */
void ox_gemv(const float *x, const ox_linear *l, float *c, int epi, float alpha);

/* --- row ops --------------------------------------------------------------------------------- */
/* LayerNorm eps 1e-5 of rows [rows][cols] (src/cpu/ops.rs:68-110); with table != NULL also the
 * NEOX split-half rotation per head of head_dim into yr, table [rows][cos(hd/2) | sin(hd/2)]. */
void ox_layer_norm(const float *x, const float *w, const float *b, float *y, int rows, int cols,
                   const float *table, float *yr, int head_dim);
/* conv1d columns, rows of ch*kernel (src/cpu/ops.rs:114-131); `width` >= ch*kernel pads rows with
 * zeros (the GPU's im2col pads to 32, src/gpu/ops.wgsl:97-119). */
void ox_im2col(const float *x, int t, int ch, int kernel, int stride, int pad, float *col,
               int width);
/* Conformer conv module middle (src/cpu/ops.rs:137-182): h [t][2ch] (GLU done in place into its
 * first halves), taps [kernel][ch], y [t][ch].  mask: NULL or the valid frame count per row
 * block (batched/padded windows: frames >= valid get a zero GLU output, as
 * src/ane/conformer.rs:301-309 multiplies by the frame mask). */
void ox_conv_glu(float *h, const float *taps, const float *tb, int kernel, const float *g,
                 const float *beta, int layer_norm, float *y, int t, int ch, int valid);
/* Multi-head attention (src/cpu/ops.rs:190-221): q at qk[i*ld + h*hd], k at qk[i*ld + ch + h*hd],
 * v at v[i*ldv + h*hd]; o [t][ch].  valid < t masks keys >= valid (additive key mask,
 * src/ane/mod.rs:463-466). */
void ox_attention(const float *qk, int ld, const float *v, int ldv, float *o, int t, int heads,
                  int hd, int valid);
/* Transformer-XL relative attention (src/cpu/ops.rs:228-273): qkv [t][q|k|v], pos
 * [2t+15][ch] (row r = position t+15-r), u/v [heads][hd]. */
void ox_relative_attention(const float *qkv, const float *pos, const float *u, const float *vb,
                           float *o, int t, int heads, int hd, int valid);
/* One query per head over an f16-rounded cache (src/cpu/ops.rs:304-337); kv = K then V, each
 * [heads][cols][hd]; q rounded to f16. */
void ox_attend(const float *q, const float *kv, int cols, int n, float *o, int heads, int hd);
/* GPU cache layout (src/gpu/decode.wgsl:148-173): f16 bits; K transposed (pair i of position j at
 * word i*cols + j), then V by position (word d/2*cols + j*d/2 + i).  rows of x from src, stride
 * floats apart, each [k(d) | v(d)]. */
void ox_pack(const float *x, int src, int stride, uint32_t *cache, int rows, int d, int cols,
             int col);
/* Rotary tables: GigaAM (src/gigaam/mod.rs:86-97) per frame [cos(hd/2) | sin(hd/2)], f64 -> f32. */
void ox_rope_table(int frames, int hd, double theta, float *out);
/* Relative positions (src/conformer.rs:144-153): rows of [sin, cos] pairs from position first
 * down. */
void ox_rel_positions(int d, long first, int rows, float *out);
/* BatchNorm fold (src/conformer.rs:132-139). */
void ox_batch_norm(const float *w, const float *b, const float *mean, const float *var, int d,
                   float *scale, float *shift);

/* --- Parakeet subsampling (src/parakeet/cpu.rs:103-174) ------------------------------------ */
/* conv0 + ReLU then conv2 into rows 2*t0-1.. of a chunk: y [rows][half(half(mels))][ch]. */
void ox_sub_first(const float *mel, int valid, int mels, const float *w0, const float *b0,
                  const float *w2, const float *b2, int ch, float *y, int rows, int t0);
/* depthwise 3x3 s2 p1 + bias over image [t][f][ch]; x holds rows 2*t0-1..; y [n][half(f)][ch]. */
void ox_depthwise(const float *x, const float *w, const float *b, int t, int f, int ch, float *y,
                  int n, int t0);
/* [t][f][ch] -> [t][ch*f] */
void ox_flatten(const float *x, float *y, int t, int f, int ch);

/* --- decoders on encoder output ------------------------------------------------------------- */
int ox_argmax(const float *v, int n); /* first maximum (src/parakeet/decoder.rs:150-158) */
/* Greedy CTC (src/gigaam/decoder.rs:135-151); returns pairs count, out [2*frames]. */
int ox_ctc(const float *logits, int frames, int classes, int blank, uint32_t *out);
/* TDT greedy control flow (src/parakeet/decoder.rs:158-191) over scripted decisions: used to pin
 * the loop against the reference's own unit tests.  script[2*i] = token, [2*i+1] = duration idx. */
int ox_tdt_scripted(int frames, int blank, const int *durations, int max_symbols, int global,
                    const int *script, int script_len, uint32_t *out, int *calls, int *used);

/* --- model level (oracle/models.c) ---------------------------------------------------------- */
typedef struct ox_model ox_model;
/* Loads a GGUF file written by wavo_amd.synth (gigaam / parakeet / whisper architectures). */
ox_model *ox_model_load(const char *path, char *err, size_t errlen);
void ox_model_free(ox_model *m);
/* Encoder output of `mel` [mel_frames][mels]: frames and width written; out NULL asks for sizes. */
int ox_model_encode(ox_model *m, const float *mel, int mel_frames, int valid, float *out,
                    int *frames, int *width);
/* Conformer blocks only, over x [t][d] in place (for layer-level checks); layers = how many. */
int ox_model_blocks(ox_model *m, float *x, int t, int layers);
int ox_model_info(ox_model *m, int *arch, int *d, int *layers, int *mels, int *width);
/* TDT greedy decode (Parakeet) of an encoder output; returns token count, (token, frame) pairs. */
int ox_model_tdt(ox_model *m, const float *enc, int frames, int width, uint32_t *out, int cap);
/* The same, recording per decision (frame, token, duration index) in trace_frame[3i..3i+2] and the
 * smaller top-2 gap of its token/duration logits in trace_gap[i] (first trace_cap decisions). */
int ox_model_tdt_trace(ox_model *m, const float *enc, int frames, int width, uint32_t *out, int cap,
                       int *trace_frame, float *trace_gap, int trace_cap);
/* One predictor step (Decoder::predict, src/parakeet/decoder.rs:107-133): token < 0 feeds zeros; state
 * and next [layers][h | c] of hidden values each; pred [joint] = the joint's predictor projection. */
int ox_model_predict(ox_model *m, int token, const float *state, float *next, float *pred);
/* The joint's logits (src/parakeet/decoder.rs:135-142): ReLU(enc_row + pred) times the output layer
 * plus its bias, [classes + durations]. */
int ox_model_joint(ox_model *m, const float *enc_row, const float *pred, float *logits);
/* max_i Σ_j |W_ij| of the joint's output layer (the logits' sensitivity to the encoder row). */
float ox_model_tdt_lipschitz(ox_model *m);
/* Whisper: cross cache from encoder output, one decoder step's logits. */
int ox_whisper_begin(ox_model *m, const float *enc, int frames);
int ox_whisper_step(ox_model *m, int token, int pos, float *logits);

/* Whisper's greedy window search (oracle/search.c; src/whisper/search.rs).  Token ids as the
 * reference's `Ids` (src/whisper/search.rs:16-23, loaded by src/whisper/mod.rs:131-141). */
typedef struct ox_whisper_ids {
  int eot, no_timestamps, begin, sot;
  const int *suppress;
  int n_suppress;
  const int *begin_suppress;
  int n_begin_suppress;
} ox_whisper_ids;
/* The model's ids (pointers into the model); -1 if it is not a Whisper model. */
int ox_model_whisper_ids(ox_model *m, ox_whisper_ids *ids);
/* The decoder's context (max_target_positions). */
int ox_model_context(ox_model *m);
/* timestamp_rules (src/whisper/search.rs:73-111), in place. */
void ox_timestamp_rules(const ox_whisper_ids *ids, float *logits, int vocab, const uint32_t *gen, int n);
/* argmax, the first maximum, and with logprob its log-softmax (src/whisper/search.rs:113-127). */
int ox_whisper_argmax(const float *logits, int vocab, int logprob, float *lp);
/* decode's `pick` (src/whisper/search.rs:46-59): suppression, begin suppression before the first
 * token, the timestamp rules, argmax; in place. */
int ox_whisper_pick(const ox_whisper_ids *ids, float *logits, int vocab, const uint32_t *gen, int n, int logprob,
                    float *lp);
/* probability (src/whisper/search.rs:129-135). */
float ox_probability(const float *logits, int vocab, int id);
/* search::decode (src/whisper/search.rs:35-71) from the logits of the prompt's last token (modified
 * in place), stepping the model (ox_whisper_step) from position `prompt`: generated ids without EOT
 * into out (count returned, -1 on error); the average log-probability in *avg when logprobs; with
 * gaps != NULL the top-2 gap of each pick after the rules (gaps[i] for the pick of out[i]). Stops
 * at EOT, 256 new tokens or position min(448, context). */
int ox_whisper_decode(ox_model *m, const ox_whisper_ids *ids, float *logits, int vocab, int prompt, int logprobs,
                      uint32_t *out, int cap, float *avg, float *gaps);
/* The margin of a pick: the two largest logits left by the rules (+inf with fewer than two). */
float ox_top2_gap(const float *logits, int vocab, const ox_whisper_ids *ids, const uint32_t *gen, int n);
/* retrieve (src/whisper/search.rs:137-181): segments as (start in 20 ms steps, first index, end
 * index) triples of gen in seg[3i..]; their text is the ids < eot in that range.  Returns the count;
 * *advance = mel frames the next window moves on. */
int ox_whisper_retrieve(const ox_whisper_ids *ids, const uint32_t *gen, int n, int frames, int *seg, int cap,
                        int *advance);

int ox_threads(void);
void ox_set_threads(int n);

/* --- log-mel frontends (oracle/frontend.c) ------------------------------------------------------ */
/* Fft::forward (src/fft.rs:72-104) of n real values: f64 (f64 != 0) or f32 arrays. */
int ox_fft(int n, int f64, const void *x, void *re, void *im);
/* Fft::new's tables (src/fft.rs:47-70): perm [n], leaf cos/sin [leaf][leaf], per stage the twiddles
 * [stages][n / 2]; any pointer may be NULL. */
int ox_fft_tables(int n, int *perm, double *leaf_cos, double *leaf_sin, double *tw_cos, double *tw_sin,
                  int *leaf, int *stages);
/* Parakeet (src/parakeet/frontend.rs): the Slaney filterbank [128][257]; log_mel of frames [t0, t1);
 * compute: [samples / 160 + 1][128] normalized (returns the frame count, 0 below 3 frames; out NULL
 * returns the count only). */
void ox_parakeet_filterbank(float *out);
int ox_parakeet_log_mel(const float *pcm, int samples, int t0, int t1, float *out);
int ox_parakeet_mel(const float *pcm, int samples, float *out);
/* GigaAM (src/gigaam/frontend.rs) and Whisper (src/whisper/frontend.rs) with the GGUF's window and
 * filterbank [mels][n_fft / 2 + 1]; out NULL returns the frame count only. */
int ox_gigaam_mel(const float *pcm, int samples, const float *window, const float *filters, int mels, float *out);
int ox_whisper_mel(const float *pcm, int samples, const float *window, const float *filters, int mels, float *out);
/* on != 0: the frontends write each filter's sum before the logarithm and skip the normalization or
 * scaling (Whisper's silent frames 0). */
void ox_mel_raw(int on);

#ifdef __cplusplus
}
#endif
#endif
