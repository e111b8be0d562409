/*
 * tiledattn.h — C ABI of the MI355X (gfx950) SDPA forward operator.
 *
 * This library is the drop-in boundary for the reference's launch path.  It replaces:
 *   - the torch op declared in torch-ext/torch_binding.h:5 and registered in
 *     torch-ext/torch_binding.cpp:6-19 (device guard + current stream + launch,
 *     tiledattention_cuda/tiledattention.cu:29-32), and
 *   - the kernel launch ct.launch(stream, grid, kernel, (q_bh, k_t, v_bh, out_bh, scale))
 *     at src/tiledattention/kernels/flash_fwd.py:809 with its arguments built at :954-969,
 *   - the in-memory kernel cache src/tiledattention/kernels/compile_cache.py:10-37
 *     (here: a per-device cache of hipFunction_t loaded from precompiled gfx950 code objects).
 *
 * Conventions:
 *   - Plain C types only; no torch or HIP types cross the boundary.  `stream` is a
 *     hipStream_t passed as void* (NULL = the device's null stream).
 *   - The library never allocates or frees device memory; the caller owns q, k, v and o.
 *   - Calls are asynchronous with respect to the host (work is enqueued on `stream`).
 *   - Every entry point returns a ta_status; on a non-OK status ta_last_error() returns a
 *     message for the calling thread.  No C++ exception crosses the boundary.
 *   - Thread-safe: the kernel cache is guarded by a mutex, and a launch resolves its kernel
 *     and enqueues it under that mutex, so ta_cache_reset / ta_set_code_object_dir never
 *     unload a module a concurrent launch is using (launches from several threads
 *     serialize for the few microseconds of the enqueue).
 */
#ifndef TILEDATTN_H_
#define TILEDATTN_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TA_ABI_VERSION 6

typedef enum ta_status {
  TA_OK = 0,
  TA_EINVAL = 1,        /* bad argument (null pointer, shape, stride, alignment, tile) */
  TA_EUNSUPPORTED = 2,  /* valid request this build has no kernel for (head dim, device arch) */
  TA_ENOKERNEL = 3,     /* code object or kernel symbol could not be loaded */
  TA_EHIP = 4           /* HIP runtime error (launch failure, bad device or stream) */
} ta_status;

typedef enum ta_dtype { TA_FP16 = 0, TA_BF16 = 1 } ta_dtype;

/* Accumulation of the P.V product across key tiles: fp32, or the input dtype
 * (TILEDATTN_ACCUM_MODE=fp16 in the reference, flash_fwd.py:123-146). */
typedef enum ta_accum { TA_ACC_FP32 = 0, TA_ACC_INPUT = 1 } ta_accum;

/* Arguments of one SDPA forward.  Mirrors what flash_fwd.py:954-956 hands to the kernel:
 * q, k, v, out as [B,H,S,D] views plus the resolved scale; the reference's [B*H,D,S] K
 * transpose view is not needed because the kernel reads K row-major. */
typedef struct ta_fwd_args {
  const void* q; /* [B,H,S,D] device pointers, dtype elements */
  const void* k;
  const void* v;
  void* o;
  int64_t B, H, S, D; /* D: 64, 96, 128, 160 or 256 (callers zero-pad other head dims,
                         or set d_real); 160 and 256 need tile_n = 64, 96 fp32
                         accumulation */
  int64_t q_stride[4]; /* element strides for (B,H,S,D); stride[3] must be 1, the others
                          non-negative multiples of 8; the row stride stride[2] at least
                          the row width (D, or d_real when set: rows must not overlap)
                          and below 2^23; S * stride[2] * 2 bytes below 2^31 for k and v
                          (and for q on the eight-wave kernels: fp32 accumulation with
                          tiles (128, 64) / (128, 128), D <= 160, or (64, 64) / (64, 128),
                          D = 64, 96 or 128, or (64, 64), D = 160), which are read with
                          32-bit buffer offsets */
  int64_t k_stride[4];
  int64_t v_stride[4];
  int64_t o_stride[4];
  float scale;     /* softmax scale, already resolved (sdpa.py:46-47) */
  int32_t causal;  /* 0/1 */
  int32_t dtype;   /* ta_dtype */
  int32_t tile_m;  /* query rows per workgroup: 64 or 128 (TILEDATTN_TILE_M) */
  int32_t tile_n;  /* keys per tile: 64 or 128 (TILEDATTN_TILE_N) */
  int32_t accum;   /* ta_accum */
  int32_t device;  /* HIP device ordinal the pointers and stream belong to */
  int32_t sched;   /* workgroup -> tile order: 0 plain, 1 XCD-grouped (causal grids of two
                      or more workgroups per CU on tiles (128, 64) / (128, 128) with fp32
                      accumulation then run query blocks in pairs nq - 1 - j and j, one
                      workgroup each), 2 XCD-grouped with causal heavy/light complementary
                      order, 3 as 1 with pairs whatever the grid size */
  int32_t d_real;  /* 0, or the head-dim columns q/k/v/o actually have (a multiple of 8 below
                      D): the kernel for D reads the missing columns as zero and does not
                      write them, so a narrower head dim needs no padded copies (the
                      reference pads on the host, flash_fwd.py:868-872).  The eight-wave
                      kernels only (fp32 accumulation; tiles (128, 64) and (128, 128) with
                      D <= 160, tiles (64, 64) and (64, 128) with D = 64, 96 or 128, tile
                      (64, 64) with D = 160). */
  int32_t aligned; /* 1: the kernel variant without tail masking runs when S is a multiple
                      of tile_m and tile_n, and on the eight-wave kernels of their 128-key
                      step (the reference's aligned fast path,
                      flash_fwd.py:199-238, 880-921); 0: the tail-masked variant always
                      runs (TILEDATTN_DISABLE_ALIGNED_FASTPATH).  Both give the same
                      result on such S; zero-initialised arguments get the masked one. */
} ta_fwd_args;

/* Version of this ABI (TA_ABI_VERSION). */
int ta_abi_version(void);

/* Directory holding the attn_fwd_m<TM>_n<TN>.hsaco code objects.  Must be called before
 * the first launch; a later call also drops every cached module. */
ta_status ta_set_code_object_dir(const char* dir);

/* Load (or find in the cache) the kernel for one configuration on `device` without
 * launching it: the counterpart of compile_cache.get_kernel's miss path
 * (compile_cache.py:13-29).  `aligned` = 1 selects the variant without tail masking,
 * valid only when S is a multiple of tile_m and tile_n. */
ta_status ta_prepare(int32_t device, int32_t dtype, int32_t head_dim, int32_t tile_m,
                     int32_t tile_n, int32_t causal, int32_t accum, int32_t aligned);

/* Enqueue one SDPA forward on `stream`.  Picks the unmasked-tail kernel when
 * args->aligned is 1 and S is a multiple of both tiles (and of 128 on the eight-wave
 * kernels, see `aligned`).  Zero-size problems (B*H == 0 or
 * S == 0) return TA_OK with no launch. */
ta_status ta_sdpa_fwd(const ta_fwd_args* args, void* stream);

/* Split key ranges: no counterpart in the reference, whose grid is one program per
 * (query block, b*h) (flash_fwd.py:806-809).  With few (b, h) slices, or causal rows whose
 * lengths differ by S / 128 key steps, that grid leaves compute units idle while the
 * longest rows finish.  The split path cuts every 128-row query block's keys into chunks of
 * `chunk_steps` steps of 128 keys, runs one workgroup per chunk, and merges the chunks of a
 * block (log-sum-exp weights) in a second kernel on the same stream.  It exists for tiles
 * (128, 64) and (128, 128) with fp32 accumulation and D <= 160; the result matches ta_sdpa_fwd within
 * fp32 rounding of the merge. */

/* Chunk length of the paired split, for causal grids of at most one workgroup per compute
 * unit: query blocks p and nq - 1 - p (nq blocks a head) share two workgroups, the second
 * block's key range cut so that each workgroup runs about (nq + 1) / 2 key steps (the
 * whole-row grid's longest runs nq); the cut blocks are merged as above.  The grid keeps
 * the whole-row size.  A non-causal call with it is exactly ta_sdpa_fwd. */
#define TA_SPLIT_PAIRS (-1)

/* Chunk length (key steps, or TA_SPLIT_PAIRS) this library would use for `args` on its
 * device: 0 when the unsplit grid is as fast (large grids, configurations without a split
 * kernel).  Computed
 * from a model of the dispatch of the grid over the device's compute units; cached per
 * (S, B*H, causal, CU count).  Reads only the shape, dtype, tile, accum and device fields
 * (tensor pointers and strides may be unset). */
ta_status ta_split_plan(const ta_fwd_args* args, int32_t* chunk_steps);

/* The model behind ta_split_plan for a device with `compute_units` CUs, without touching
 * a device: chunk length (or TA_SPLIT_PAIRS) for a 128-row-tile fp32-accumulation forward
 * of sequence length S over n_bh (b, h) slices, 0 for no split or invalid sizes. */
int32_t ta_split_plan_model(int64_t S, int64_t n_bh, int32_t causal, int32_t compute_units);

/* The same for blocks of `rows` query rows (128: the model above; 64: the 64-row kernel's
 * chunks, planned for grids whose 64-row blocks fill at most half of the compute units and
 * where the wide kernel does not run, TA_LAYOUT_WIDE) at kernel head dim `head_dim`; 0 for
 * no split. */
int32_t ta_split_plan_model_rows(int64_t S, int64_t n_bh, int32_t causal, int32_t head_dim, int32_t rows,
                                 int32_t compute_units);

/* Device workspace (bytes, 256-byte aligned base required) that ta_sdpa_fwd_split needs
 * for `chunk_steps`; 0 when that chunk length splits nothing.  Needs no device; reads only
 * the shape, dtype, tile and accum fields. */
ta_status ta_split_workspace_size(const ta_fwd_args* args, int32_t chunk_steps, int64_t* bytes);

/* Enqueue one SDPA forward with split key ranges on `stream`.  chunk_steps = 0, or a
 * chunk length that splits nothing, is exactly ta_sdpa_fwd.  The workspace is owned by the
 * caller, needs no initialisation, and must not be used by another call until this one's
 * work on `stream` has finished.  The split blocks are merged by the split kernel itself
 * (ta_launch_desc.merge_in_kernel) with arrival counters the library keeps per (device,
 * stream) in the code object, or, past 16 streams on a device, by a merge kernel on
 * `stream` after it.  Every launch leaves its counters at zero, so a launch captured in a
 * HIP graph replays as it ran (it keeps the capture stream's counter region: its replays
 * must not overlap a split launch on that stream). */
ta_status ta_sdpa_fwd_split(const ta_fwd_args* args, int32_t chunk_steps, void* workspace,
                            int64_t workspace_bytes, void* stream);

/* Bytes of the static split workspace of ta_sdpa_fwd_split_static, per device. */
#define TA_STATIC_SCRATCH_BYTES (64LL << 20)

/* ta_sdpa_fwd_split with the workspace in a static device array of
 * TA_STATIC_SCRATCH_BYTES held by each GPU the library runs on, so that the call allocates
 * no device memory.  No counterpart in the reference: it is for callers that cannot call
 * hipMalloc (code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation).  Same arguments, kernels and result as ta_sdpa_fwd_split; a chunk length
 * whose workspace (ta_split_workspace_size) exceeds TA_STATIC_SCRATCH_BYTES is rejected
 * with TA_EINVAL, and a chunk length that splits nothing runs ta_sdpa_fwd (no scratch).
 * Every call on one GPU shares that GPU's array: calls whose work overlaps on the same GPU
 * (other streams, other threads) race on it and must be serialized by the caller.  The
 * first call on a device resolves the array's address there (hipGetSymbolAddress, which
 * loads the library's device code on that device) and loads the code object of its
 * kernels: make one call on each device before capturing a graph or entering code that must
 * not allocate; later calls allocate nothing. */
ta_status ta_sdpa_fwd_split_static(const ta_fwd_args* args, int32_t chunk_steps, void* stream);

/* How a forward's work is laid out over workgroups (ta_launch_desc.layout). */
typedef enum ta_layout {
  TA_LAYOUT_WHOLE_ROWS = 0,   /* one workgroup per query block of `rows` rows */
  TA_LAYOUT_PAIRS = 1,        /* causal query blocks nq - 1 - j and j on one workgroup */
  TA_LAYOUT_ROWS256 = 2,      /* non-causal 256-row blocks (the two wave groups own
                                 different rows) */
  TA_LAYOUT_SPLIT = 3,        /* chunks of key steps, merged by a second kernel */
  TA_LAYOUT_PAIRED_SPLIT = 4, /* the paired split (TA_SPLIT_PAIRS), merged likewise */
  TA_LAYOUT_WIDE = 5          /* 32-row blocks whose eight waves split the keys of every
                                 pass (64-row tiles on grids of one round of the CUs) */
} ta_layout;

/* What one forward enqueues: the kernels, their grids and code object, and the decisions
 * behind them.  Filled by ta_describe_launch from the same planning step the launch entry
 * points run, so a description and the launch it describes cannot differ. */
typedef struct ta_launch_desc {
  char code_object[64];   /* file of the kernels ("" when nothing is launched) */
  char kernel[96];        /* the attention kernel's symbol */
  int64_t grid;           /* its workgroups (0: zero-size problem, nothing launched) */
  int32_t block;          /* its threads per workgroup */
  int32_t rows;           /* query rows per query block it processes (32, 64, 128 or 256) */
  int32_t tail;           /* 1: the tail-masked variant */
  int32_t layout;         /* ta_layout */
  int32_t chunk_steps;    /* the split that runs: 0 whole rows, > 0 chunk length, or
                             TA_SPLIT_PAIRS */
  int32_t compute_units;  /* compute units the decision was made for */
  char merge_kernel[96];  /* the merge kernel of a split ("" when none) */
  int64_t merge_grid;
  int32_t merge_block;
  int32_t in_place_pad;   /* 1: the kernel family reads d_real < D in place (eight-wave) */
  int32_t split_capable;  /* 1: split kernels exist for this configuration */
  int32_t merge_in_kernel; /* 1: the split kernel merges its blocks itself (the last
                              workgroup to finish a block combines its partials), so the
                              merge kernel runs only when the launching stream finds no
                              free counter region (more than 16 streams launching splits) */
  int64_t workspace_bytes; /* workspace ta_sdpa_fwd_split needs for chunk_steps (0 if none) */
} ta_launch_desc;

/* Describe what ta_sdpa_fwd (chunk_steps = 0) or ta_sdpa_fwd_split (chunk_steps != 0)
 * would enqueue for `args` on its device, without launching anything.  No counterpart in
 * the reference, whose single kernel is fixed by its tile knobs (flash_fwd.py:895-952):
 * here the pairs, 256-row and split layouts are chosen from the grid size and the
 * device's compute units, and callers that label or model launches (benchmarks,
 * profilers, schedulers) read the choice from the library instead of restating its rules.
 * Reads the shape, dtype, tile, accum, causal, sched, aligned, d_real and device fields
 * (tensor pointers and strides may be unset). */
ta_status ta_describe_launch(const ta_fwd_args* args, int32_t chunk_steps, ta_launch_desc* out);

/* ta_describe_launch for a device with `compute_units` CUs, without touching a device. */
ta_status ta_describe_launch_model(const ta_fwd_args* args, int32_t chunk_steps,
                                   int32_t compute_units, ta_launch_desc* out);

/* Chunk length meaning "the library's dispatch model decides" (TILEDATTN_SPLIT=auto). */
#define TA_SPLIT_AUTO (-2)

/* Knob values of one call, as the TILEDATTN_* environment knobs or an operator's arguments
 * give them. */
typedef struct ta_call_knobs {
  int32_t tile_m, tile_n; /* both 0: the default rule; else the tile, 64 or 128 each */
  int32_t accum;          /* -1 auto (fp32 on gfx950), TA_ACC_FP32 or TA_ACC_INPUT */
  int32_t aligned;        /* 1: the aligned fast path is allowed; 0: disabled */
  int32_t sched;          /* -1: the default order; 0..3 as ta_fwd_args.sched */
  int32_t split;          /* TA_SPLIT_AUTO, 0 (whole rows), a chunk length or TA_SPLIT_PAIRS */
} ta_call_knobs;

/* What one call runs: the launch arguments (all but q, k, v, o, the strides and scale,
 * which the caller fills) and what the caller does around the launch. */
typedef struct ta_call_plan {
  ta_fwd_args args;        /* shape (D = the kernel's head dim), dtype, causal, tiles, accum,
                              device, sched, d_real, aligned */
  int32_t chunk_steps;     /* 0: ta_sdpa_fwd; else ta_sdpa_fwd_split with this chunk length */
  int32_t host_pad;        /* zero columns the caller appends to q, k and v (0: none) */
  int32_t out_width;       /* columns of the output buffer (the caller's head dim, or the
                              kernel's when padded on the host: slice it back) */
  int32_t reserved;
  int64_t workspace_bytes; /* device workspace of the split (0: none) */
} ta_call_plan;

/* The host policy of one forward of q, k, v [B, H, S, D] (the reference's
 * run_flash_fwd up to its launch, flash_fwd.py:821-969): tile (the knob or the default
 * rule), accumulation, kernel head dim and padding (in the kernel where it can, else on
 * the host), the aligned fast path, workgroup order and split key ranges.  compute_units
 * 0 reads the device's count; a positive value plans for such a device without touching
 * one.  No counterpart in the reference's C++ (its policy is Python); the library's torch
 * operator and any non-Python caller plan through it, and the Python package applies the
 * same rules. */
ta_status ta_plan_call(int64_t B, int64_t H, int64_t S, int64_t D, int32_t dtype, int32_t causal,
                       int32_t device, int32_t compute_units, const ta_call_knobs* knobs,
                       ta_call_plan* out);

/* Unload every cached module on every device (compile_cache.reset_cache_for_tests). */
ta_status ta_cache_reset(void);

/* Number of kernels currently cached (all devices). */
int32_t ta_cache_size(void);

/* Message for the last non-OK status returned on the calling thread ("" if none). */
const char* ta_last_error(void);

/* Static name of a status code. */
const char* ta_status_string(int32_t status);

#ifdef __cplusplus
}
#endif

#endif /* TILEDATTN_H_ */
