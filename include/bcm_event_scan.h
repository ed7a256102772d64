/*
 * bcm_event_scan.h - C ABI of the MI355X (gfx950) event-sparse selective-scan
 * library (libbcm_event_scan.so).
 *
 * The library implements BC_mamba's event path in three stages, each with a
 * forward and a backward:
 *   1. event extraction  : dense membrane -> per-channel event streams
 *   2. flat selective scan over the packed events (depthwise B/C mode)
 *   3. zero-order-hold restore of event outputs to a dense (B, L, D) tensor
 *
 * Conventions (all entry points):
 *   - every pointer is a device pointer unless stated otherwise; the caller
 *     allocates every input, output and workspace buffer; the library never
 *     allocates device memory and holds no state other than a thread-local
 *     error string, the process-wide scan-family setting
 *     (bcm_set_scan_family) and the scratch of the allocation-free entry
 *     point, so calls on different streams may run concurrently;
 *   - work is enqueued on `stream` (a hipStream_t; NULL = default stream) of
 *     the current device; no entry point synchronises the host;
 *   - the return value is BCM_OK or an error code; bcm_last_error() returns
 *     a message that starts with the entry point's name;
 *   - dtype codes: BCM_F32 / BCM_F16 / BCM_BF16 (the reference accepts the
 *     same three for u / z / out / dout / membrane / restore in and out);
 *   - index tensors (channel ids, time steps, gaps k, cu_seqlens) are int32,
 *     channel-major (channel = b * D + d), time-ascending inside a channel.
 *
 * Internal event index (produced by bcm_extract_fill or
 * bcm_build_event_index, consumed by restore and the row-wise gather
 * backward): a bitmask [rows, bcm_bitmask_words(L)] of uint32 words (bit t%32
 * of word t/32 set iff an event at step t) and a tile table
 * [channels, bcm_tile_count(L) + 1] of int32 holding, for every 64-step tile,
 * the absolute index of the channel's first event at or after the tile start.
 */
#ifndef BCM_EVENT_SCAN_H
#define BCM_EVENT_SCAN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BCM_ABI_VERSION 4

typedef struct ihipStream_t* bcm_stream_t; /* == hipStream_t */

enum bcm_dtype { BCM_F32 = 0, BCM_F16 = 1, BCM_BF16 = 2, BCM_U8 = 3 /* bool / byte membrane only */ };
enum bcm_status { BCM_OK = 0, BCM_EINVAL = 1, BCM_EHIP = 2 };

/* ---- library ------------------------------------------------------------ */
int bcm_abi_version(void);
const char* bcm_last_error(void);
/* words per bitmask row for sequence length L (a multiple of 32) */
int64_t bcm_bitmask_words(int64_t L);
/* number of 64-step tiles per row: ceil(L / 64) */
int64_t bcm_tile_count(int64_t L);
/* zero `bytes` bytes at `ptr` with a fill kernel (no hipMemset: graph-safe) */
int bcm_zero(void* ptr, int64_t bytes, bcm_stream_t stream);

/* ---- (1) event extraction ----------------------------------------------- */
/* Pass 1 of extract_base_events (csrc/extract/extract_events_cuda.cu:192-208
 * count_base_kernel): event = float(membrane[row, t]) > threshold (strict).
 * membrane [n_rows, L] of `dtype` (BCM_U8 reads a bool/byte mask, used by the
 * legacy extract_events with threshold 0.5); writes bitmask [n_rows, words]
 * and counts [n_rows]. */
int bcm_extract_count(const void* membrane, int dtype, int64_t n_rows,
                      int64_t L, float threshold, uint32_t* bitmask,
                      int32_t* counts, bcm_stream_t stream);

/* Pass 2 (extract_events_cuda.cu:361-372, DeviceScan + cu[0]=0 + counts.max):
 * cu_seqlens[0] = 0, cu_seqlens[i+1] = sum(counts[0..i]);
 * meta[0] = total events E, meta[1] = max(counts) (0 when n_rows == 0).
 * meta (8-byte aligned) may be device memory or pinned (hipHostMalloc'd,
 * device-mapped) host memory. Both values land in one 64-bit store written
 * through to memory, so a host that set meta[0] = -1 beforehand may poll it
 * (no event, no copy): once meta[0] >= 0, meta[1] is valid too. */
int bcm_extract_scan(const int32_t* counts, int64_t n_rows,
                     int32_t* cu_seqlens, int32_t* meta, bcm_stream_t stream);

/* Pass 3 (extract_events_cuda.cu:226-312 fill_base_kernel, fused with
 * expand_events_direct_kernel :482-509 and gather_events_fwd2_kernel
 * :629-642). Emits the events of every base row c into the `expand` logical
 * channels c*expand + r at positions base_cu[c]*expand + r*count_c + i:
 * k_flat (k = t+1 for a channel's first event, else the gap to the previous
 * event) and, unless NULL, ch_ids and t_steps (a consumer that works from
 * the bitmask and tile table needs neither). Optional (NULL to skip): x
 * [n_rows*expand, L] of
 * x_dtype gathered at the events into x_events [E*expand]; tile_start
 * [n_rows*expand, tile_count+1]; head_flags [E*expand] (1 at a channel's
 * first event, else 0: the legacy extract_events output, :102-114). */
int bcm_extract_fill(const uint32_t* bitmask, const int32_t* base_cu,
                     int64_t n_rows, int64_t L, int64_t expand,
                     const void* x, int x_dtype, int32_t* ch_ids,
                     int32_t* t_steps, int32_t* k_flat, void* x_events,
                     int32_t* tile_start, int32_t* head_flags,
                     bcm_stream_t stream);

/* Passes 1-3 without a separate offsets pass (no reference counterpart: it
 * replaces the DeviceScan of extract_events_cuda.cu:361-372 in the fused
 * model path, one kernel fewer).
 * bcm_extract_count_blocks: as bcm_extract_count; each block of 4 rows also
 * writes its rows' event sum and maximum count to block_sums (int32, of
 * bcm_extract_block_sums_bytes: nblk sums, nblk maxima, nblk + 1 words of
 * scratch, nblk = ceil(n_rows/4)).
 * bcm_extract_fill_blocks: as bcm_extract_fill, each block deriving its
 * rows' offsets from block_sums and counts (for more than 4096 blocks a
 * one-workgroup scan of the block sums into the scratch words runs first,
 * so the offset work stays linear in n_rows); it writes cu_seqlens
 * [n_rows*expand+1] (logical channels) and meta = (E_base, max count) as
 * bcm_extract_scan does (one 64-bit store written through to memory: a host
 * that set meta[0] = -1 may poll pinned meta while the fill runs). Since E
 * is not known when the fill is enqueued, its event outputs must be sized
 * for every possible event (n_rows*expand*L). ch_ids, t_steps, x / x_events
 * and tile_start are optional (NULL to skip). */
int64_t bcm_extract_block_sums_bytes(int64_t n_rows);
int bcm_extract_count_blocks(const void* membrane, int dtype, int64_t n_rows,
                             int64_t L, float threshold, uint32_t* bitmask,
                             int32_t* counts, int32_t* block_sums,
                             bcm_stream_t stream);
int bcm_extract_fill_blocks(const uint32_t* bitmask, const int32_t* counts,
                            const int32_t* block_sums, int32_t* meta,
                            int64_t n_rows, int64_t L, int64_t expand,
                            const void* x, int x_dtype, int32_t* cu_seqlens,
                            int32_t* ch_ids, int32_t* t_steps,
                            int32_t* k_flat, void* x_events,
                            int32_t* tile_start, bcm_stream_t stream);

/* The straight-through spike head that produces the next block's membrane
 * (SpikeSamplerSurrogate mode "ste", e_model.py:233-254, lra_impl.py:1398;
 * p = sigmoid(prob_head(...)) [B, L, Dm]) emitting the event bitmask
 * directly: bitmask row b * Dm + d gets bit t set where p[b, t, d] >= threshold
 * (the rows of bcm_extract_count over the transposed spikes, whose strict
 * "> thr_extract" with 0 <= thr_extract < 1 selects exactly these steps).
 * With s_out != NULL also writes the spike value s = (p >= threshold) + p - p
 * in p's dtype and layout, rounded as torch evaluates it. The padding words
 * of each bitmask row are not written. */
int bcm_spike_bits(const void* p, int dtype, int64_t B, int64_t L, int64_t Dm, float threshold,
                   uint32_t* bitmask, void* s_out, bcm_stream_t stream);
/* counts and block_sums of bcm_extract_count_blocks from a finished bitmask
 * (bcm_spike_bits), for bcm_extract_fill_blocks(_conv). */
int bcm_extract_count_bits(const uint32_t* bitmask, int64_t n_rows, int64_t L, int32_t* counts,
                           int32_t* block_sums, bcm_stream_t stream);

/* bcm_extract_fill_blocks with the depthwise causal conv + SiLU of the
 * model block (e_model.py:442-451) evaluated at the events instead of
 * gathered from a dense x_conv (the conv producer fused with the gather,
 * e_model.py:403-406): for the event (ch, t), d = ch % dim,
 *   x_events[e] = silu(bias[d] + sum_k weight[d,k] x[ch, t-(K-1)+k])
 * with x = 0 before t = 0 (plain conv when silu == 0); the value, rounding
 * included, that bcm_causal_conv1d_fwd writes at (ch, t). x is the conv
 * input: row ch = b * dim + d starts at x + b * x_batch_stride +
 * d * x_dim_stride (elements; rows contiguous), so the [D, B*L] output of the
 * in_proj GEMM is read in place. weight [dim, K] (K <= 8), bias [dim] or
 * NULL, fp32. The other arguments are those of bcm_extract_fill_blocks. */
int bcm_extract_fill_blocks_conv(const uint32_t* bitmask, const int32_t* counts,
                                 const int32_t* block_sums, int32_t* meta,
                                 int64_t n_rows, int64_t L, int64_t expand,
                                 const void* x, int x_dtype, int64_t x_batch_stride,
                                 int64_t x_dim_stride, int64_t dim, const float* weight,
                                 const float* bias, int K, int silu, int32_t* cu_seqlens,
                                 int32_t* ch_ids, int32_t* t_steps, int32_t* k_flat,
                                 void* x_events, int32_t* tile_start, bcm_stream_t stream);

/* expand_base_events (extract_events_cuda.cu:529-603): logical cu_seqlens
 * [n_rows*expand+1] and expanded streams [E_base*expand]. */
int bcm_expand_events(const int32_t* base_ch, const int32_t* base_t,
                      const int32_t* base_k, const int32_t* base_cu,
                      int64_t n_rows, int64_t E_base, int64_t expand,
                      int32_t* ch_ids, int32_t* t_steps, int32_t* k_flat,
                      int32_t* cu_seqlens, bcm_stream_t stream);

/* out[0] = max_i (cu[i+1] - cu[i]) over n channels (extract_events_cuda.cu
 * :598-600 diff.max()); 0 when n == 0. */
int bcm_seqlen_max(const int32_t* cu_seqlens, int64_t n, int32_t* out,
                   bcm_stream_t stream);

/* gather_events_fwd (extract_events_cuda.cu:670-708):
 * out[e] = x[ch_ids[e] * L + t_steps[e]], x viewed as [rows, L]. */
int bcm_gather_fwd(const void* x, int dtype, int64_t n_rows, int64_t L,
                   const int32_t* ch_ids, const int32_t* t_steps, int64_t E,
                   void* out, bcm_stream_t stream);

/* gather_events_bwd (extract_events_cuda.cu:717-754): dx [n_rows, L] = 0
 * except dx[ch_ids[e], t_steps[e]] = g[e]; (ch, t) pairs must be unique. */
int bcm_gather_bwd(const void* g, int dtype, const int32_t* ch_ids,
                   const int32_t* t_steps, int64_t E, int64_t n_rows,
                   int64_t L, void* dx, bcm_stream_t stream);

/* Same result as bcm_gather_bwd for channel-major sorted streams, written
 * row by row from the event index (no zero pass, no scatter). The bitmask
 * row of channel ch is ch / mask_row_div. */
int bcm_gather_bwd_rows(const void* g, int dtype, const uint32_t* bitmask,
                        int64_t mask_row_div, const int32_t* tile_start,
                        int64_t n_rows, int64_t L, void* dx,
                        bcm_stream_t stream);

/* ---- (2) flat per-channel selective scan -------------------------------- */
/* Argument block of the depthwise flat_ch scan; mirrors SSMParamsFlatSeg /
 * SSMParamsFlatSegBwd (csrc/selective_scan/selective_scan.h:151-283) minus
 * the fields that the flat_ch path never reads. Set unused pointers to NULL.
 *   Δ_i   = dt_idle[d]*(k_i-1) + dt_active[d],  d = ch % dim
 *   a_i,s = exp2(clamp(Δ_i*A[d,s]*log2(e), -126, 126))
 *   h_i,s = a_i,s*h_{i-1},s + Δ_i*u_i*(u_i*W_B[d,s])
 *   y_i   = D[d]*u_i + sum_s h_i,s*(u_i*W_C[d,s]);  out_z = y*silu(z)   */
typedef struct bcm_scan_args {
  int64_t n_events;    /* E */
  int32_t n_channels;  /* NC = len(cu_seqlens) - 1 */
  int32_t dim;         /* A.shape[0] */
  int32_t dstate;      /* A.shape[1], <= 256 */
  int32_t max_seqlen;  /* max events per channel */
  int32_t n_chunks;    /* max(1, ceil(max_seqlen / 2048)) */
  int32_t dtype;       /* dtype of u, z, out, out_z, dout, du, dz */
  const void* u;               /* [E] */
  const int32_t* k;            /* [E] */
  const int32_t* cu_seqlens;   /* [NC + 1] */
  const float* dt_idle;        /* [dim] */
  const float* dt_active;      /* [dim] */
  const float* A;              /* [dim, dstate] */
  const float* W_B;            /* [dim, dstate] */
  const float* W_C;            /* [dim, dstate] */
  const float* D;              /* [dim] or NULL */
  const void* z;               /* [E] or NULL */
  /* forward outputs */
  void* out;                   /* [E] ungated y */
  void* out_z;                 /* [E] y * silu(z), when z != NULL */
  float* x;                    /* [NC, n_chunks, 2*dstate]: (prod a, h) */
  /* backward inputs */
  const void* dout;            /* [E] */
  const float* x_saved;        /* [NC, n_chunks, 2*dstate] from forward */
  const void* out_saved;       /* [E] ungated forward output (z only) */
  /* backward outputs (fully written, no zero-init needed) */
  void* du;                    /* [E] */
  float* dA;                   /* [dim, dstate] */
  float* dW_B;                 /* [dim, dstate] */
  float* dW_C;                 /* [dim, dstate] */
  float* ddt_idle;             /* [dim] */
  float* ddt_active;           /* [dim] */
  float* dD;                   /* [dim] or NULL */
  void* dz;                    /* [E] when z != NULL */
  /* [NC, n_pass, dstate] state h at the start of every pass of a channel
   * (pass 0 unused), n_pass from bcm_scan_chunking. The forward
   * writes it when non-NULL; the backward needs it when the pass is shorter
   * than 2048 events (n_pass > 1 and pass_len < 2048), else it re-seeds
   * from x_saved as the reference does. */
  float* chunk_g;
  int64_t chunk_g_bytes;       /* size of chunk_g (checked: too small is an error) */
  /* backward workspace of bcm_scan_bwd_workspace_bytes(args) bytes, or
   * NULL: with it, model channels with many channels each are split over
   * several workgroups whose parameter-gradient partials are summed in a
   * fixed order (same results either way up to that order). */
  float* split_ws;
  int64_t split_ws_bytes;      /* size of split_ws (too small: no split) */
  /* Optional (NULL: not reported) int32 status word, device memory or
   * device-mapped pinned host memory, that the caller zeroes beforehand.
   * The kernels set it to BCM_SCAN_SEQLEN_EXCEEDED when some channel holds
   * more than max_seqlen events: x and chunk_g are sized from max_seqlen,
   * so such a channel's saved states (and with them the backward of its
   * later passes, and bcm_scan_bwd_rows' dense row) are incomplete. Every
   * write stays inside the buffers either way. bcm_scan_bwd_rows may also
   * set BCM_SCAN_ROWS_INCOMPLETE (see below). */
  int32_t* status;
  /* Events per pass that chunk_g is laid out for: the pass_len that
   * bcm_scan_chunking returned when the caller sized chunk_g (the forward
   * that fills it and the backward that reads it each check it against
   * their own pass length: a mismatch, e.g. a forward and a backward run
   * under different scan families, is BCM_EINVAL, as the reference refuses
   * a stale chunk count, selective_scan.cpp:1009-1014). Ignored when chunk_g
   * is NULL. */
  int32_t chunk_g_pass;
  /* Optional (NULL: not used) [E] float32, depthwise mode: the forward's
   * per-event state sum acc_i = sum_s W_B[d,s] W_C[d,s] g_i,s (so that
   * y_i = D u_i + u_i acc_i, with g = h / W_B). A forward given it writes
   * it; a backward given it reads it instead of rebuilding the sums from
   * the saved states (the caller hands the backward what the forward of the
   * same inputs wrote). No counterpart in the reference, which recomputes. */
  float* acc;
} bcm_scan_args;

#define BCM_SCAN_SEQLEN_EXCEEDED 1
/* bcm_scan_bwd_rows only: the dense rows were left incomplete because a row
 * writer stopped waiting for the scan waves (a bounded wait that correct
 * runs never reach; reported rather than risking a wave that never ends). */
#define BCM_SCAN_ROWS_INCOMPLETE 2

/* Which kernel family runs a depthwise scan, for the whole process:
 * BCM_SCAN_AUTO picks by shape (the state lanes of dstate 16 from one wave
 * of four channels per SIMD up, the lane groups otherwise),
 * BCM_SCAN_LANES / BCM_SCAN_ITEMS force the state lanes (dstate 16) / the
 * lane groups. The initial value comes from the environment variable
 * BCM_SCAN_KERNEL ("lanes", "items"; read once, at the first scan call),
 * else BCM_SCAN_AUTO. The family fixes chunk_g's pass length, so a forward
 * and its backward must run under the same setting (chunk_g_pass checks
 * it). Returns the previous setting, or -1 for an unknown code. No
 * counterpart in the reference (it has one kernel family). */
enum bcm_scan_family { BCM_SCAN_AUTO = 0, BCM_SCAN_LANES = 1, BCM_SCAN_ITEMS = 2 };
int bcm_set_scan_family(int family);

/* Events per pass of a channel (pass_len) and passes of the longest channel
 * (n_pass) for these arguments (max_seqlen, n_events, n_channels, dstate):
 * channels longer than one pass carry their state between passes. Returns
 * BCM_OK; *needs_chunk_g = 1 when the backward must be given chunk_g. */
int bcm_scan_chunking(const bcm_scan_args* args, int32_t* pass_len, int32_t* n_pass,
                      int32_t* needs_chunk_g);
/* Bytes of bcm_scan_args.split_ws for a backward with these arguments (0:
 * no split, split_ws may stay NULL). */
int64_t bcm_scan_bwd_workspace_bytes(const bcm_scan_args* args);
/* selective_scan_fwd_flat_ch, depthwise mode (selective_scan.cpp:674-884,
 * selective_scan_fwd_kernel.cuh:403-728). */
int bcm_scan_fwd(const bcm_scan_args* args, bcm_stream_t stream);
/* selective_scan_bwd_flat_ch, depthwise mode (selective_scan.cpp:890-1153,
 * selective_scan_bwd_kernel.cuh:635-1169). */
int bcm_scan_bwd(const bcm_scan_args* args, bcm_stream_t stream);

/* The model path's scan backward with the gather backward folded in
 * (SelectiveScanFlatChFn.backward then GatherEventsFn.backward, e_model.py
 * :188-193, extract_events_cuda.cu:717-754): everything bcm_scan_bwd
 * writes (du included), plus dx [n_channels, seqlen] (args->dtype) = du at
 * each channel's events and 0 elsewhere, the result of bcm_gather_bwd_rows
 * on du. bitmask / tile_start are the extraction's event index
 * (bcm_extract_indexed) and must describe the events of cu_seqlens. One
 * kernel for single-pass 16-lane shapes without z and seqlen % 4 == 0
 * (dx aligned to 4 elements); otherwise the two steps run in turn. When it
 * runs as one kernel (bcm_scan_bwd_rows_fused), args->du may be NULL: dx
 * then holds the only copy of du (a caller that needs only dx, as the
 * model's backward, skips the du stream); in the two-step case a NULL du
 * is BCM_EINVAL. */
typedef struct bcm_scan_rows {
  const uint32_t* bitmask;    /* [n_channels / mask_row_div, words], 8-byte aligned */
  int64_t mask_row_div;       /* channel ch reads bitmask row ch / mask_row_div */
  const int32_t* tile_start;  /* [n_channels, tiles + 1] */
  int64_t seqlen;             /* L */
  void* dx;                   /* [n_channels, L] */
} bcm_scan_rows;
int bcm_scan_bwd_rows(const bcm_scan_args* args, const bcm_scan_rows* rows, bcm_stream_t stream);
/* 1 when bcm_scan_bwd_rows(args, rows) runs as one kernel (and so accepts a
 * NULL args->du), 0 when it runs the two steps, negative for invalid
 * arguments. Enqueues nothing. No counterpart in the reference. */
int bcm_scan_bwd_rows_fused(const bcm_scan_args* args, const bcm_scan_rows* rows);

/* B and C of the non-depthwise modes of fwd_flat_ch / bwd_flat_ch
 * (selective_scan.cpp:760-776, 840-848, 969-990, 1085-1090):
 *   BCM_BC_LEGACY  per event: B[s*b_row_stride + e]  ([dstate, E])
 *                  per model channel: B[s*b_row_stride + d]  ([dstate, dim])
 *   BCM_BC_TILED   per event: B[((tile_offsets[ch] + p/T)*dstate + s)*T + p%T]
 *                  for the event at position p of channel ch, T =
 *                  tile_chunk_size; tiles outside [0, n_tiles) read 0.
 * C alike. The recurrence is h_i = a_i h_{i-1} + B_i Δ_i u_i and
 * y_i = D u_i + Σ_s C_i h_i (W_B / W_C of bcm_scan_args are not read). */
enum bcm_bc_layout { BCM_BC_LEGACY = 1, BCM_BC_TILED = 2 };
typedef struct bcm_scan_bc {
  int32_t layout;           /* bcm_bc_layout */
  int32_t b_per_event;      /* legacy: 1 = [dstate, E], 0 = [dstate, dim]; tiled: 1 */
  int32_t c_per_event;
  int32_t tile_chunk_size;  /* tiled: T >= 1 */
  int64_t b_row_stride;     /* legacy: elements between the rows of B */
  int64_t c_row_stride;
  int64_t n_tiles;          /* tiled: leading dimension of B and C */
  const int32_t* tile_offsets;  /* tiled: [n_channels] first tile of each channel */
  const float* B;
  const float* C;
  /* backward outputs, the layouts of B and C. Per-event entries are written
   * for every event; tiled entries that no event maps to are not written
   * (zero-fill them); per-model-channel entries are fully written. */
  float* dB;
  float* dC;
  int64_t db_row_stride;    /* legacy */
  int64_t dc_row_stride;
} bcm_scan_bc;

/* selective_scan_fwd_flat_ch with legacy or tiled B/C (selective_scan.cpp
 * :760-776, selective_scan_fwd_kernel.cuh:566-686). Outputs as bcm_scan_fwd. */
int bcm_scan_var_fwd(const bcm_scan_args* args, const bcm_scan_bc* bc, bcm_stream_t stream);
/* Workspace of bcm_scan_var_bwd: the forward states, 4*E*dstate bytes. */
int64_t bcm_scan_var_workspace_bytes(int64_t n_events, int dstate);
/* selective_scan_bwd_flat_ch with legacy or tiled B/C (selective_scan.cpp
 * :969-990, selective_scan_bwd_kernel.cuh:902-1112): du, dA, ddt_*, dD, dz
 * in args; dB and dC in bc. Recomputes the forward states into the
 * workspace first (x_saved is not read). */
int bcm_scan_var_bwd(const bcm_scan_args* args, const bcm_scan_bc* bc, void* workspace,
                     int64_t workspace_bytes, bcm_stream_t stream);

/* ---- causal depthwise conv1d (+ SiLU): the producer of x_conv ---------- */
/* e_model.py:442-451 (silu(conv1d(x)[..., :L]), groups = channels, padding
 * K-1; or causal_conv1d_fn(x, w, bias, activation="silu")). x, out:
 * [B, D, L] contiguous (dtype); weight [D, K] and bias [D] fp32 (bias may be
 * NULL); K <= 8. silu = 0 gives the plain convolution. */
int bcm_causal_conv1d_fwd(const void* x, int dtype, const float* weight, const float* bias, int64_t B,
                          int64_t D, int64_t L, int K, int silu, void* out, bcm_stream_t stream);
/* Backward: dx [B, D, L] (dtype), dweight [D, K] and dbias [D] (fp32, fully
 * written; dbias may be NULL), the SiLU derivative recomputed from x. With a
 * workspace of bcm_causal_conv1d_bwd_workspace_bytes bytes the batch rows
 * of a channel are split over several workgroups (partials summed in a
 * fixed order); with NULL one workgroup per channel takes all of them. */
int64_t bcm_causal_conv1d_bwd_workspace_bytes(int64_t B, int64_t D, int64_t L, int K);
int bcm_causal_conv1d_bwd(const void* x, int dtype, const float* weight, const float* bias, const void* dout,
                          int64_t B, int64_t D, int64_t L, int K, int silu, void* dx, float* dweight,
                          float* dbias, void* workspace, int64_t workspace_bytes, bcm_stream_t stream);

/* Backward of the conv evaluated at the events (bcm_extract_fill_blocks_conv)
 * and the gather (GatherEventsFn.backward, e_model.py:188-193, then the conv
 * backward of e_model.py:442-451): from du [n_events], the gradient of
 * x_events, with g = du * silu'(pre) at the events and 0 elsewhere,
 *   dx[ch, t] = sum_k weight[d,k] g[ch, t+(K-1)-k]   (dtype; every step written)
 *   dweight[d,k] = sum g x[ch, t-(K-1)+k],  dbias[d] = sum g   (fp32, fully
 *   written; rows summed in row order, no atomics)
 * x and dx have the row strides of bcm_extract_fill_blocks_conv (rows
 * ch = b * D + d, B * D of them); bitmask / mask_row_div / tile_start are
 * the extraction's event index. Needs L and both strides multiples of 4,
 * x and dx aligned to 4 elements, and a workspace of
 * bcm_causal_conv1d_bwd_events_workspace_bytes(B, D, K) bytes. */
int64_t bcm_causal_conv1d_bwd_events_workspace_bytes(int64_t B, int64_t D, int K);
int bcm_causal_conv1d_bwd_events(const void* x, int dtype, int64_t x_batch_stride, int64_t x_dim_stride,
                                 int64_t B, int64_t D, int64_t L, const float* weight, const float* bias,
                                 int K, int silu, const void* du, int64_t n_events,
                                 const uint32_t* bitmask, int64_t mask_row_div,
                                 const int32_t* tile_start, void* dx, float* dweight, float* dbias,
                                 void* workspace, int64_t workspace_bytes, bcm_stream_t stream);

/* ---- (3) zero-order-hold restore ---------------------------------------- */
/* Event index of sorted per-channel time steps (the restore kernels' input
 * when the caller has no bitmask): bitmask [n_rows, words], tile_start
 * [n_rows, tiles+1]. Steps outside [0, L) are ignored. If zero_f32 != NULL,
 * zero_f32[0 .. n_zero) is set to 0 (zero-init of the restore backward). */
int bcm_build_event_index(const int32_t* t_steps, const int32_t* cu_seqlens,
                          int64_t n_rows, int64_t L, uint32_t* bitmask,
                          int32_t* tile_start, float* zero_f32,
                          int64_t n_zero, bcm_stream_t stream);

/* restore_dense_fwd (csrc/r_nodecay/restore_dense.cpp:43-130,
 * restore_dense_fwd_kernel.cuh:38-114): out[b, t, d] = y[e] for the last
 * event e of channel b*dim+d with t_e <= t, 0 before the first event.
 * y holds n_events values; out (n_rows/dim, L, dim) of out_dtype is fully
 * written. */
int bcm_restore_fwd(const void* y, int y_dtype, int64_t n_events,
                    const uint32_t* bitmask,
                    int64_t mask_row_div, const int32_t* tile_start,
                    int64_t n_rows, int64_t dim, int64_t L, void* out,
                    int out_dtype, bcm_stream_t stream);

/* Workspace of bcm_restore_bwd: 3 * 4 * n_rows * tile_count(L) bytes. */
int64_t bcm_restore_bwd_workspace_bytes(int64_t n_rows, int64_t L);

/* restore_dense_bwd (restore_dense.cpp:138-202,
 * restore_dense_bwd_kernel.cuh:42-112): dy[e] = sum of dout[b, t, d] over
 * t in [t_e, t_next) (t_next = next event or L), float32. Every event with
 * 0 <= t_e < L is written exactly once (no zero-init, no atomics,
 * deterministic); `workspace` holds per-tile partial sums and end indices. */
int bcm_restore_bwd(const void* dout, int dtype, const uint32_t* bitmask,
                    int64_t mask_row_div, const int32_t* tile_start,
                    int64_t n_rows, int64_t dim, int64_t L, float* dy,
                    int64_t n_events, void* workspace,
                    int64_t workspace_bytes, bcm_stream_t stream);

/* Allocation-free variant of bcm_restore_bwd. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments, checks and result as bcm_restore_bwd, without
 * the workspace: the per-tile partials live in the library's own scratch,
 * a static device array of 8 MiB per device, so n_rows * ceil(L / 64) must
 * not exceed BCM_RESTORE_BWD_NOALLOC_MAX_TILES (checked; larger problems
 * are refused with BCM_EINVAL). It calls no hipMalloc / hipFree. All calls
 * on one device share that device's scratch: calls that overlap in time on
 * one device (different streams, no ordering between them) race and must
 * not be issued; calls in one stream are ordered and safe. Nothing in the
 * scratch needs clearing between calls (the tile pass writes every entry
 * the fix-up pass reads). */
#define BCM_RESTORE_BWD_NOALLOC_MAX_TILES 699040
int bcm_restore_bwd_noalloc(const void* dout, int dtype, const uint32_t* bitmask,
                            int64_t mask_row_div, const int32_t* tile_start,
                            int64_t n_rows, int64_t dim, int64_t L, float* dy,
                            int64_t n_events, bcm_stream_t stream);

/* Sync area of bcm_restore_bwd_chained: 8 * (2 + n_rows * tile_count(L))
 * bytes. */
int64_t bcm_restore_bwd_sync_bytes(int64_t n_rows, int64_t L);

/* restore_dense_bwd (restore_dense.cpp:138-202,
 * restore_dense_bwd_kernel.cuh:42-112) in one kernel: the result of
 * bcm_restore_bwd (every event with 0 <= t_e < L written exactly once, no
 * atomics on dy), with the runs that cross 64-step tile edges closed by a
 * look-back over the preceding tiles' published partials instead of a
 * second pass. Sums within a run follow a different order than
 * bcm_restore_bwd where a run crosses two or more tile edges (fp32
 * rounding; equal otherwise). dy_dtype: BCM_F32 (the reference's dy), or
 * dout's 16-bit dtype: the fp32 sums rounded to nearest even as stored,
 * the cast the reference's autograd applies to dy before the scan
 * backward (e_model.py's RestoreDenseFn feeding SelectiveScanFlatChFn).
 * `sync` (8-byte aligned, sync_bytes >= bcm_restore_bwd_sync_bytes) must
 * be zero before its first use; every call that completes leaves it zero
 * again, so a caller zeroes it once and reuses it. Word 1 (uint64) becomes
 * nonzero if a wait gave up, which consistent inputs never cause; the area
 * must then be zeroed again. Calls that share a sync area must be ordered
 * (one stream); calls with separate areas may overlap. */
int bcm_restore_bwd_chained(const void* dout, int dtype, const uint32_t* bitmask,
                            int64_t mask_row_div, const int32_t* tile_start,
                            int64_t n_rows, int64_t dim, int64_t L, void* dy,
                            int dy_dtype, int64_t n_events, void* sync,
                            int64_t sync_bytes, bcm_stream_t stream);

/* ---- (3') restore -> out_proj ------------------------------------------- */
/* The block's restore followed by its output projection (e_model.py:499-504:
 * y_dense = restore_dense_fn(y_flat, ...); out = self.out_proj(y_dense)),
 * without the dense restore output: out[b, t, :] = weight z[b, t, :] + bias
 * with z[b, t, d] the zero-order hold of bcm_restore_fwd. fp32 throughout;
 * weight is the nn.Linear weight [d_model, dim] (row-major), bias [d_model]
 * or NULL, out (n_rows/dim, L, d_model) is fully written. n_events * 4 must
 * stay below 2 GiB. */
int bcm_restore_proj_fwd(const float* y, int64_t n_events, const uint32_t* bitmask,
                         int64_t mask_row_div, const int32_t* tile_start,
                         int64_t n_rows, int64_t dim, int64_t L,
                         const float* weight, const float* bias, int64_t d_model,
                         float* out, bcm_stream_t stream);

/* Workspace of bcm_restore_proj_bwd: the restore backward's per-tile
 * arrays (3 * 4 * n_rows * tile_count(L)) and the weight gradient's
 * partials (4 * d_model * dim per (sequence, 512-step segment)). A call
 * with dweight == NULL needs only the per-tile arrays (the size of
 * bcm_restore_bwd_workspace_bytes(n_rows, L)). */
int64_t bcm_restore_proj_bwd_workspace_bytes(int64_t n_rows, int64_t dim, int64_t L,
                                             int64_t d_model);

/* Backward of bcm_restore_proj_fwd (the out_proj backward of the
 * reference's nn.Linear, then RestoreDenseFn.backward, e_model.py:146-157,
 * restore_dense_bwd_kernel.cuh:42-112), from dout (n_rows/dim, L, d_model):
 *   dy[e]   = sum over t in [t_e, t_next) of (dout[b, t, :] . weight[:, d]),
 *             float32, every event written once (no zero-init, no atomics);
 *   dweight = sum over (b, t) of dout[b, t, :] (x) z[b, t, :], [d_model, dim]
 *             (fully written; partials summed in a fixed order).
 * dy or dweight may be NULL to skip it; y is needed for dweight. The bias
 * gradient (the column sums of dout) is not computed here. */
int bcm_restore_proj_bwd(const float* dout, const float* y, int64_t n_events,
                         const uint32_t* bitmask, int64_t mask_row_div,
                         const int32_t* tile_start, int64_t n_rows, int64_t dim,
                         int64_t L, const float* weight, int64_t d_model, float* dy,
                         float* dweight, void* workspace, int64_t workspace_bytes,
                         bcm_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* BCM_EVENT_SCAN_H */
