/*
 * gaussfield.h - C ABI of libgaussfield.so, the MI355X (gfx950) Gaussian-field
 * weight-delta renderer.
 *
 * A layer's delta-W (out_features x in_features, fp32, row-major) is the sum of K
 * anisotropic 2-D Gaussians, binned into tile_out x tile_in tiles by their
 * sigma_multiplier-sigma bounding boxes.  Every pointer argument is a device
 * pointer unless its name ends in _host.  Every entry point returns 0 on success
 * and a non-zero GF_E* code otherwise; gf_last_error() then holds the message
 * (thread-local).  `stream` is a hipStream_t (NULL = the legacy default stream).
 *
 * Reference interface replaced (Plutohr/GUASS, paths under gaussian_peft/cuda_field):
 *   csrc/ext.cpp:9-37     gaussian_field_forward           -> gf_forward_bin(_info) + gf_forward_render
 *   csrc/ext.cpp:38-72    gaussian_field_backward          -> gf_backward_train (or gf_backward)
 *   csrc/ext.cpp:73-110   gaussian_field_backward_reference-> gf_backward (same gradients)
 *   csrc/field.h:11-18    ForwardConfig                    -> gf_field_config
 *   csrc/field_impl.cu:52-108 input / saved-state checks   -> GF_E_* codes + device-side checks
 */
#ifndef GAUSSFIELD_H_
#define GAUSSFIELD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GF_OK 0
#define GF_E_INVALID_ARGUMENT 1   /* bad size / config (tile_out<=0, sigma<=0, ...)      */
#define GF_E_WORKSPACE 2          /* workspace missing or smaller than *_workspace_bytes  */
#define GF_E_HIP 3                /* a HIP runtime call or kernel launch failed           */
#define GF_E_CAPACITY 4           /* pair count exceeds the gaussian_ids capacity         */
#define GF_E_SAVED_STATE 5        /* saved tile_ptr / gaussian_ids violate the contract   */
#define GF_E_INTERNAL 6           /* device-side consistency check failed                 */

/* Device-side status bits, written to the status word by the kernels (see gf_read_status). */
#define GF_STATUS_CAPACITY 0x1u        /* more pairs than ids_capacity: ids truncated        */
#define GF_STATUS_COUNT_MISMATCH 0x2u  /* per-tile counts disagree with per-Gaussian sums    */
#define GF_STATUS_TILE_PTR_LAST 0x4u   /* backward: tile_ptr[T] != number of pairs           */
#define GF_STATUS_TILE_PTR_ORDER 0x8u  /* render / backward: tile_ptr decreasing / below 0 / outside [0, pairs] */
#define GF_STATUS_IDS_NEGATIVE 0x10u   /* backward: a gaussian id < 0                        */
#define GF_STATUS_IDS_RANGE 0x20u      /* backward: a gaussian id >= K                       */

/* Mirrors ForwardConfig (reference csrc/field.h:11-18). */
typedef struct gf_field_config {
  int64_t tile_out;          /* tile height in rows of delta-W, > 0                         */
  int64_t tile_in;           /* tile width in columns of delta-W, > 0                       */
  double sigma_multiplier;   /* bounding-box half-width in standard deviations, > 0         */
  int32_t normalize;         /* non-zero: multiply each Gaussian by 1/(2*pi*sqrt(det cov))  */
  int32_t has_clamp_quad;    /* non-zero: clamp the quadratic form to [0, clamp_quad]       */
  double clamp_quad;         /* upper clamp of the quadratic form (80.0 in the layer)       */
} gf_field_config;

/* Library / device facts. */
const char* gf_version(void);
const char* gf_last_error(void);

/* Tile grid of an out_features x in_features delta-W (reference forward.cu:29-35). */
int gf_tile_grid(int64_t out_features, int64_t in_features, const gf_field_config* cfg,
                 int64_t* num_tile_rows_host, int64_t* num_tile_cols_host);

/* Workspace sizes in bytes (device memory the caller provides, 256-byte aligned).  The
 * backward workspace must be zero-filled before its first use; gf_backward leaves it zeroed
 * again, so a workspace kept across calls needs one clear at allocation. */
size_t gf_forward_workspace_bytes(int64_t out_features, int64_t in_features, int64_t k,
                                  const gf_field_config* cfg);
size_t gf_backward_workspace_bytes(int64_t out_features, int64_t in_features, int64_t k,
                                   const gf_field_config* cfg);
/* The largest gf_forward_workspace_bytes over every k in [0, k_capacity] (it is not monotone in
 * k: past the mask path's limit the coverage masks drop out).  A workspace of this size serves
 * any k up to the capacity, so densified fields (reference controllers/clone.py:31-56,
 * prune.py:34-45) change k without reallocating.  No reference counterpart (the reference
 * allocates its workspaces per call, field_impl.cu:110-133); 0 on an invalid argument. */
size_t gf_forward_workspace_bytes_max(int64_t out_features, int64_t in_features, int64_t k_capacity,
                                      const gf_field_config* cfg);

/*
 * Forward phase 1 (binning): per-Gaussian geometry and sigma-box tile ranges, per-tile
 * Gaussian counts and their exclusive scan.  For 16x16 or 32x32 tiles with 1 <= k <= 8192 (the
 * mask path) it also stores every Gaussian's evaluation constants and, per tile row and tile
 * column, a bitmask of the Gaussians whose tile range covers it; the render then reads each
 * tile's ids from those masks and gf_forward_emit has nothing to do.  Where the render bins the
 * tiles itself -- the mask path with k <= 256 (and k * T <= 2^23), each tile by its wave, and
 * single 16x16 fields with k <= 1024 (C < 2^15, k * T < 2^31), each tile row by a render
 * workgroup -- no masks are stored, and tile_ptr and num_pairs_dev are written by
 * gf_forward_render (num_pairs_host, when given, is still P, summed on the host from
 * per-workgroup counts in the workspace header).
 *   amp             [K,1] fp32 (read on the mask path; may be NULL otherwise)
 *   tile_ptr        [T+1] int64 out: tile t owns gaussian_ids_sorted[tile_ptr[t] : tile_ptr[t+1]]
 *   num_pairs_dev   [1] int64 out: P = tile_ptr[T] = sum over Gaussians of tiles touched
 *   num_pairs_host  optional: if non-NULL the call synchronises `stream` and stores P here
 *                   (the only host synchronisation in the forward, as reference forward.cu:48-73).
 * Replaces reference forward.cu:372-511 (preprocess_geometry + build_binning_state up to tile_ptr).
 */
int gf_forward_bin(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                   const float* mu, const float* chol_raw, const float* amp,
                   int64_t* tile_ptr, int64_t* num_pairs_dev, int64_t* num_pairs_host,
                   void* workspace, size_t workspace_bytes, void* stream);

/* What the binning learnt of a field, for the host. */
typedef struct gf_bin_info {
  int64_t num_pairs; /* P */
  int64_t max_span;  /* the most tiles one Gaussian's tile rectangle covers (0 for K = 0) */
} gf_bin_info;

/*
 * gf_forward_bin with the read-back of P widened to gf_bin_info (the same one synchronisation
 * and copy).  max_span decides between the one-launch backward and the reduction + finish
 * (gf_backward_train, gf_backward_direct): one Gaussian over many tiles serialises the one-launch
 * kernel's atomics on its gradient slot.  info must not be NULL.
 */
int gf_forward_bin_info(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                        const float* mu, const float* chol_raw, const float* amp, int64_t* tile_ptr,
                        int64_t* num_pairs_dev, gf_bin_info* info, void* workspace, size_t workspace_bytes,
                        void* stream);

/* gf_bin_info of the last forward on a forward workspace (gf_forward, gf_forward_bin + _render,
 * gf_fwd_bwd_fused, the capacity-mode forward), after that forward in `stream` order:
 * synchronises `stream`. */
int gf_read_bin_info(const void* forward_workspace, gf_bin_info* info, void* stream);

/*
 * Forward phase 2 (emission; returns at once on the mask path): writes the (tile, gaussian)
 * pairs into gaussian_ids_sorted, each tile's ids inside its [tile_ptr[t], tile_ptr[t+1]) range
 * (order fixed by phase 3), and stores each Gaussian's evaluation constants in the workspace
 * (from the covariance gf_forward_bin left there, with amp applied).  Must follow
 * gf_forward_bin on the same stream with the same workspace, tile_ptr and mu.
 *   gaussian_ids_sorted [ids_capacity] int64 out; pairs beyond the capacity are dropped and
 *                   GF_STATUS_CAPACITY is set
 * Replaces reference forward.cu:465-482 (emit_tile_pairs_kernel + radix sort on the tile key).
 */
int gf_forward_emit(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                    const float* mu, const float* amp, const int64_t* tile_ptr,
                    int64_t* gaussian_ids_sorted, int64_t ids_capacity,
                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * Forward phase 3 (render): puts every tile's ids in canonical order (gaussian id ascending;
 * with tile-major ranges this is the (tile, gaussian) order of a stable sort) and renders
 * delta-W from the Gaussian constants stored by gf_forward_emit (or, on the mask path,
 * gf_forward_bin, in which case the render writes the ids itself from the masks).  Must follow
 * gf_forward_emit on the same stream with the same workspace and ids.
 *   tile_ptr        [T+1] int64, from gf_forward_bin; written here instead where the render
 *                   bins the tiles itself (with P to gf_forward_bin's num_pairs_dev): the mask
 *                   path with k <= 256 and k * T <= 2^23, and single 16x16 fields with
 *                   k <= 1024, C < 2^15 and k * T < 2^31 (a workgroup per tile row)
 *   delta           [out_features*in_features] fp32 out, row-major; every element written
 * Replaces reference forward.cu:513-569 (tile_accumulate_kernel; delta needs no pre-zeroing).
 */
int gf_forward_render(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                      const float* row_coords, const float* col_coords, int64_t* tile_ptr,
                      int64_t* gaussian_ids_sorted, int64_t ids_capacity,
                      float* delta, void* workspace, size_t workspace_bytes, void* stream);

/*
 * The whole forward in one call, without a host synchronisation: gf_forward_bin +
 * gf_forward_emit + gf_forward_render into a gaussian-id buffer of fixed capacity (pairs past it
 * are dropped and GF_STATUS_CAPACITY is set; P goes to num_pairs_dev), for callers that keep
 * their buffers, e.g. under HIP graph capture.  The capacity also sizes the launch of the
 * heavy-tile workgroups: past it, on a field with such workgroups, tiles of more than 24
 * Gaussians beyond the bound are left unrendered.  GF_STATUS_CAPACITY asks for a larger capacity
 * either way; tile_ptr and P are complete.  Replaces reference field_impl.cu:135-163
 * (gaussian_field_forward, which reads P back to size its id buffer).
 */
int gf_forward(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
               const float* row_coords, const float* col_coords, const float* mu, const float* chol_raw,
               const float* amp, int64_t* tile_ptr, int64_t* num_pairs_dev, int64_t* gaussian_ids_sorted,
               int64_t ids_capacity, float* delta, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Backward: reduces dL/d(delta) into per-Gaussian gradients through the saved binning.
 * gf_backward = gf_backward_reduce (per-tile moments, atomics into the workspace) followed by
 * gf_backward_finish (chain rule, clears the workspace accumulators).
 *   grad_delta      [out_features*in_features] fp32
 *   tile_ptr        [T+1], int64 if tile_ptr_is_int64 else int32
 *   gaussian_ids    [num_pairs], int64 if ids_is_int64 else int32 (any order within a tile)
 *   d_mu [K,2], d_chol_raw [K,3], d_amp [K,1] fp32 out (fully written)
 *   forward_workspace  optional: the workspace of the forward over the same (mu, chol_raw)
 *                   and config (after its gf_forward_emit); the Gaussians' constants and
 *                   Cholesky factors stored there are read instead of recomputed, and the
 *                   forward's list of heavy tiles lets the reduction split them over
 *                   workgroups.  NULL recomputes them.
 * Saved-state violations (non-monotone tile_ptr, tile_ptr[T] != num_pairs, ids outside
 * [0,K)) are detected on the device, the offending pairs skipped, and status bits set.
 * Replaces reference backward.cu:541-716 (backward_pair_reduce_train).
 */
int gf_backward(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                const float* grad_delta, const float* row_coords, const float* col_coords,
                const float* mu, const float* chol_raw, const float* amp,
                const void* tile_ptr, int32_t tile_ptr_is_int64,
                const void* gaussian_ids, int32_t ids_is_int64, int64_t num_pairs,
                float* d_mu, float* d_chol_raw, float* d_amp, const void* forward_workspace,
                void* workspace, size_t workspace_bytes, void* stream);

/* First half of gf_backward (reference backward.cu:592-702: per-pair partials + reduce-by-key). */
int gf_backward_reduce(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                       const float* grad_delta, const float* row_coords, const float* col_coords,
                       const float* mu, const float* chol_raw,
                       const void* tile_ptr, int32_t tile_ptr_is_int64,
                       const void* gaussian_ids, int32_t ids_is_int64, int64_t num_pairs,
                       const void* forward_workspace, void* workspace, size_t workspace_bytes,
                       void* stream);

/* Second half of gf_backward (reference backward.cu:436-496,704-715: cov -> chol_raw chain).
 * forward_workspace as for gf_backward_reduce: optional; the forward's Cholesky factor and
 * covariance are read instead of recomputed from chol_raw. */
int gf_backward_finish(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                       const float* chol_raw, const float* amp,
                       float* d_mu, float* d_chol_raw, float* d_amp, const void* forward_workspace,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * gf_backward for the training entry (replaces reference backward.cu:541-716, the backward
 * of runtime.py:107-203's GaussianFieldCudaTrainFunction): the same arguments and outputs,
 * plus max_span, gf_bin_info.max_span of the forward that filled forward_workspace.  Where that
 * forward's binning allows it -- forward_workspace given, int64 tile_ptr and ids, max_span known
 * (>= 0) and below the one-launch limit, and a field gf_backward_direct runs in one launch -- the
 * gradients come from gf_backward_direct's kernel and one small kernel moves them into d_mu,
 * d_chol_raw, d_amp and clears the forward workspace's slots, so that a further backward on the
 * same forward starts from zero.  Otherwise it is gf_backward.  The outputs are written, not
 * added to, either way; they agree within fp32 rounding.  Two backwards on one forward workspace
 * must not run concurrently.
 */
int gf_backward_train(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                      const float* grad_delta, const float* row_coords, const float* col_coords, const float* mu,
                      const float* chol_raw, const float* amp, const void* tile_ptr, int32_t tile_ptr_is_int64,
                      const void* gaussian_ids, int32_t ids_is_int64, int64_t num_pairs, int64_t max_span,
                      float* d_mu, float* d_chol_raw, float* d_amp, void* forward_workspace, void* workspace,
                      size_t workspace_bytes, void* stream);

/*
 * gf_backward in one launch where it can (replaces reference backward.cu:541-716 like
 * gf_backward).  The chain rule is linear in the per-tile moments; the forward's first phase
 * (on the mask path) stores each Gaussian's map from moments to gradients, so the reduction
 * adds gradients instead of moments and no finish pass follows.  The gradients are ADDED into
 * the forward workspace, which every forward on it clears: from byte gf_forward_grads_offset(...)
 * of it, K slots of 8 fp32, slot g = (d_amp[g], d_mu[g][0..1], d_chol_raw[g][0..2], 2 unused)
 * (one slot per Gaussian keeps each Gaussian's atomics on one cache line).  A second call after
 * the same forward therefore leaves twice the gradients in the slots, whichever path runs;
 * callers that need one backward's gradients copy them out and run the next forward first.
 * forward_workspace is required: that of the forward over the same (mu, chol_raw, amp) and
 * config, with its int64 tile_ptr and ids (fields with heavy tiles included: their four-wave
 * workgroups add into the slots too).  Fields off the mask path and dense fields
 * (num_pairs >= 16 T) run gf_backward_reduce + gf_backward_finish, whose finish adds into the
 * same slots; so do fields whose widest tile rectangle is known (max_span >= 0,
 * gf_bin_info.max_span of the forward) to cover 320 tiles or more, where one Gaussian's atomics
 * on its one slot would cost the kernel more than the second launch (about 10 ns a tile), and
 * grids of 8192 tiles or more whose widest rectangle is not known (max_span < 0: graphs
 * captured before the content is; their reduction spreads each Gaussian's atomics over
 * stripes).  The gradients agree with gf_backward's
 * within fp32 rounding (the map is applied per tile, in fp32).
 */
int gf_backward_direct(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                       const float* grad_delta, const float* row_coords, const float* col_coords,
                       const float* mu, const float* chol_raw, const float* amp, const int64_t* tile_ptr,
                       const int64_t* gaussian_ids, int64_t num_pairs, int64_t max_span, void* forward_workspace,
                       size_t forward_workspace_bytes, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Capacity mode of gf_forward and gf_backward_direct, for graphs that must outlive a change of K
 * (densification clones and prunes Gaussians every 50-200 steps, reference
 * controllers/clone.py:31-56, prune.py:34-45, base_trainer.py:126-220; the reference re-runs its
 * whole forward per call, field_impl.cu:135-179).  k_capacity fixes everything the host decides and
 * every kernel argument -- workspace layouts (gf_forward_workspace_bytes / gf_backward_workspace_bytes
 * at k_capacity), mask words, launch grids, the kernels taken -- and the kernels read the live K
 * from k_dev (device int64, clamped to [0, k_capacity]) and the backward the live pair count from
 * num_pairs_dev (the forward's output).  A HIP graph captured over these two calls therefore stays
 * valid when *k_dev changes: the caller keeps mu [k_capacity,2], chol_raw [k_capacity,3] and
 * amp [k_capacity,1] in fixed buffers whose first *k_dev rows are the live Gaussians, and writes
 * the new K before replaying.  Outputs as gf_forward / gf_backward_direct for the live field (the
 * gradient slots of Gaussians 0 .. *k_dev - 1).  The mask path only: 16x16 or 32x32 tiles,
 * 1 <= k_capacity <= 8192; other fields are refused with GF_E_INVALID_ARGUMENT.  ids_capacity bounds
 * the pairs of every live K (pairs past it are dropped and GF_STATUS_CAPACITY is set).
 */
int gf_forward_kcap(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k_capacity,
                    const int64_t* k_dev, const float* row_coords, const float* col_coords, const float* mu,
                    const float* chol_raw, const float* amp, int64_t* tile_ptr, int64_t* num_pairs_dev,
                    int64_t* gaussian_ids_sorted, int64_t ids_capacity, float* delta, void* workspace,
                    size_t workspace_bytes, void* stream);

int gf_backward_direct_kcap(const gf_field_config* cfg, int64_t out_features, int64_t in_features,
                            int64_t k_capacity, const int64_t* k_dev, const float* grad_delta,
                            const float* row_coords, const float* col_coords, const float* mu,
                            const float* chol_raw, const float* amp, const int64_t* tile_ptr,
                            const int64_t* gaussian_ids, const int64_t* num_pairs_dev, int64_t ids_capacity,
                            void* forward_workspace, size_t forward_workspace_bytes, void* workspace,
                            size_t workspace_bytes, void* stream);

/*
 * Forward and backward in one pass, for callers that hold dL/d(delta) before the forward (fits to
 * a fixed target, benchmarks of the path): gf_forward's outputs (tile_ptr, P into num_pairs_dev,
 * the ids, delta) and gf_backward_direct's gradients (added into the forward workspace's slots at
 * gf_forward_grads_offset, which this call's binning clears first) from the binning (two launches)
 * and one tile kernel that renders delta-W and reduces grad_delta with the same exponentials.
 * Replaces reference forward.cu:372-511 (binning), then forward.cu:254-368 (tile_accumulate_kernel)
 * and backward.cu:234-388 (backward_pair_partial_kernel) run back to back on the same tiles.
 * delta agrees with gf_forward's within fp32 rounding (each pixel's Gaussians are summed as four
 * interleaved partial sums), the gradients with gf_backward_direct's; binning is identical.
 * Takes the fields gf_fwd_bwd_fused_supported accepts: 16x16 tiles on the mask path
 * (1 <= k <= 8192), fewer than 8192 tiles, sparse (ids_capacity < 16 T) and no heavy tiles; others
 * return GF_E_INVALID_ARGUMENT before any device work.  No host synchronisation.
 */
int gf_fwd_bwd_fused(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                     const float* row_coords, const float* col_coords, const float* mu, const float* chol_raw,
                     const float* amp, const float* grad_delta, int64_t* tile_ptr, int64_t* num_pairs_dev,
                     int64_t* gaussian_ids_sorted, int64_t ids_capacity, float* delta, void* forward_workspace,
                     size_t forward_workspace_bytes, void* stream);

/* 1 if gf_fwd_bwd_fused takes this field and id capacity, else 0 (also on an invalid configuration).
 * max_span as for gf_backward_direct: the one-pass kernel adds into the same slots, so a known
 * rectangle of 320 tiles or more (from an earlier step's gf_read_bin_info) answers 0; the call
 * itself reads nothing back and cannot see the widest rectangle of its own binning. */
int gf_fwd_bwd_fused_supported(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                               int64_t ids_capacity, int64_t max_span);

/* Kernel launches gf_backward_direct makes for this field, pair count and widest rectangle
 * (max_span < 0: not known): 1 (the direct kernel) or 2 (reduction + finish); the negated error
 * code on an invalid configuration. */
int gf_backward_direct_launches(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                                int64_t num_pairs, int64_t max_span);

/* Byte offset, in a forward workspace, of gf_backward_direct's gradient slots (K x 8 floats).
 * 0 on an invalid configuration. */
size_t gf_forward_grads_offset(int64_t out_features, int64_t in_features, int64_t k,
                               const gf_field_config* cfg);

/*
 * Batched fields (no single-call counterpart in the reference, which renders each adapted
 * layer separately, gaussian_linear.py:162-220; this is the batched launch of an SD1.5
 * UNet's adapted attention layers).  Every phase runs as one launch over all layers, each layer with the
 * buffers its single-field calls would use.  16x16 or 32x32 tiles (32x32 needs every layer on the
 * mask path: K <= 8192); int64 ids.
 */
typedef struct gf_layer {
  int64_t out_features, in_features, k;
  const float* row_coords;       /* [out_features] */
  const float* col_coords;       /* [in_features] */
  const float* mu;               /* [k,2] */
  const float* chol_raw;         /* [k,3] */
  const float* amp;              /* [k,1] */
  float* delta;                  /* [out_features*in_features] out */
  int64_t* tile_ptr;             /* [T+1] out */
  int64_t* num_pairs;            /* [1] out */
  int64_t* gaussian_ids;         /* [ids_capacity] out */
  int64_t ids_capacity;
  void* forward_workspace;       /* gf_forward_workspace_bytes */
  size_t forward_workspace_bytes;
  const float* grad_delta;       /* backward only: [out_features*in_features] */
  float* d_mu;                   /* backward only: [k,2] out */
  float* d_chol_raw;             /* backward only: [k,3] out */
  float* d_amp;                  /* backward only: [k,1] out */
  void* backward_workspace;      /* backward only: gf_backward_workspace_bytes, zeroed once */
  size_t backward_workspace_bytes;
  /* Launch grids and block maps are sized for max(k, k_capacity) Gaussians (0: k).  Densified
   * adapters change k every few hundred steps (reference controllers/clone.py:31-56,
   * prune.py:34-45); re-planned for any k <= k_capacity into the same plan buffer, the plan keeps
   * its gf_batch_info, so launches captured in a graph stay valid.  The buffers above must be
   * sized for the current k only. */
  int64_t k_capacity;
  /* 1: mu holds GaussianLinear's mu_raw (gaussian_linear.py:153-154 takes mu = tanh(mu_raw));
   * the kernels use tanh(mu_raw) (the device tanhf torch's GPU tanh uses) and d_mu receives
   * dL/d(mu_raw).  0: mu is used as given. */
  int32_t mu_tanh;
  int32_t reserved;
  /* Merged consumer (GaussianLinear with delta_apply "merged", reference
   * gaussian_linear.py:218-242 composes W + adapter_scale * delta-W before its GEMM).  With
   * merged_weight set, the batched render also writes merged_weight = base_weight +
   * delta_scale * delta-W, each element rounded as the fp32 product and then the fp32 sum (no FMA),
   * so it equals torch's `weight + delta * scale` bit for bit; delta may then be NULL (delta-W not
   * stored; its norm is still read back).  The backward then takes grad_delta as
   * dL/d(merged_weight) and returns the gradients of the loss through delta_scale * delta-W.
   * NULL: no merged output, grad_delta is dL/d(delta). */
  const float* base_weight;      /* [out_features*in_features], read when merged_weight is set */
  float* merged_weight;          /* [out_features*in_features] out, or NULL */
  float delta_scale;             /* finite */
  int32_t reserved2;
} gf_layer;

typedef struct gf_batch_info {
  int32_t n_layers;
  int32_t has_backward;          /* backward_buffers and every layer's grad_delta is set */
  int64_t tile_blocks, emit_blocks, finish_blocks;
  size_t plan_bytes;             /* device bytes of the plan buffer */
  int32_t backward_buffers;      /* every layer has its backward workspace and gradient outputs */
  int32_t mask_clamp;            /* clamp_quad < 80: the backward drops clamped pixels from the
                                    quadratic-form moments (at 80 and above they are below e^-40) */
  int64_t render_blocks;         /* workgroups of the tile-pair render: 4 pairs of 16x16 tiles each */
  int32_t tile_render;           /* 1: some layer renders tile by tile (32x32 tiles, or a k capacity
                                    past the masks), a second launch over the tile map */
  int32_t reserved;
} gf_batch_info;

/*
 * Builds the device plan of a batch: call with plan == NULL to get info->plan_bytes, then
 * with a device buffer of that size.  The second call copies the layer table to the device
 * and synchronises `stream`.  The plan stays valid while the layers' buffers do.
 */
int gf_batch_plan(const gf_field_config* cfg, const gf_layer* layers, int32_t n_layers, void* plan,
                  size_t plan_bytes, gf_batch_info* info, void* stream);

/* Phase selectors: GF_PHASE_ALL for a whole pass; single phases exist for timing. */
#define GF_PHASE_BIN 0x1u
#define GF_PHASE_EMIT 0x2u
#define GF_PHASE_RENDER 0x4u
#define GF_PHASE_REDUCE 0x1u
#define GF_PHASE_FINISH 0x2u
#define GF_PHASE_ALL 0xffu

/* gf_forward_bin + gf_forward_emit + gf_forward_render of every layer: three launches (two
 * when every layer is on the mask path). */
int gf_batch_forward(const void* plan, const gf_batch_info* info, uint32_t phases, void* stream);

/* gf_backward of every layer (with its pair constants): two launches. */
int gf_batch_backward(const void* plan, const gf_batch_info* info, uint32_t phases, void* stream);

/*
 * Replaces every layer's dL/d(delta) pointer in a batch plan (grad_delta: n_layers device
 * pointers, none NULL), e.g. with the gradients an autograd engine allocated for this step.
 * Asynchronous on `stream` (the pointers travel as kernel arguments; no host
 * synchronisation) and sets info->has_backward when the layers have their backward buffers.
 * A plan built with every gf_layer.grad_delta set needs no call.
 */
int gf_batch_set_grads(void* plan, gf_batch_info* info, const float* const* grad_delta, void* stream);

/*
 * Per layer of a batch plan: the forward | backward GF_STATUS_* bits (status_host), the pair
 * count of the last forward (pairs_host) and the Frobenius norm of its delta-W
 * (delta_norm_host, from per-block sums of squares the batched render leaves in the forward
 * workspace, added in double in a fixed order; the reference reads it per layer with a
 * blocking .item(), gaussian_linear.py:218); any may be NULL; clear != 0 resets the status
 * words.  One small kernel and one device-to-host copy; synchronises `stream`.
 */
int gf_batch_read(void* plan, const gf_batch_info* info, int32_t clear, uint32_t* status_host,
                  int64_t* pairs_host, double* delta_norm_host, void* stream);

/*
 * Allocation-free gf_backward.  A project-only interface with no counterpart in the reference,
 * for callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Call it once outside any capture first: that call
 * looks up this GPU's scratch address (hipGetSymbolAddress) and keeps it.
 * Same arguments and gradients as gf_backward with forward_workspace = NULL (the Gaussians'
 * constants are recomputed from mu / chol_raw), but the backward workspace is a static device
 * array of 4 MiB held by the library on each GPU it runs on until the process ends; the call
 * makes no hipMalloc / hipFree and allocates nothing else.  It covers fields whose workspace
 * (gf_backward_workspace_bytes) fits 4 MiB: K <= 131,064 below 2048 tiles (K <= 32,766 below
 * 8192 tiles, K <= 16,383 below 16,384 tiles, K <= 4,095 above); larger fields are rejected with GF_E_WORKSPACE before any
 * device work.  Each call clears the part of the array it uses (a kernel, no memset), so it
 * needs no set-up; every call on one GPU shares that GPU's array, so calls that overlap on one
 * GPU (different streams or threads without ordering) race and must be serialised by the caller.
 *   status_dev      optional [1] uint32 out (device): the call's GF_STATUS_* bits (saved-state
 *                   violations), written on `stream`; NULL skips it.
 */
int gf_backward_noalloc(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                        const float* grad_delta, const float* row_coords, const float* col_coords,
                        const float* mu, const float* chol_raw, const float* amp,
                        const void* tile_ptr, int32_t tile_ptr_is_int64,
                        const void* gaussian_ids, int32_t ids_is_int64, int64_t num_pairs,
                        float* d_mu, float* d_chol_raw, float* d_amp, uint32_t* status_dev, void* stream);

/*
 * Reads (and, if clear != 0, resets) the device status word of a workspace produced by the
 * calls above.  Synchronises `stream` for the read; a reset (needed only when a bit is set) is
 * queued on `stream` after it, ahead of any later work there.  *status_host receives
 * GF_STATUS_* bits.
 */
int gf_read_status(void* workspace, int32_t clear, uint32_t* status_host, void* stream);

/*
 * Self-test hook (no reference counterpart): evaluates on the GPU the fp32 softplus the
 * binning uses, F.softplus as the reference CPU path computes it (covariance.py:23,25),
 * over all 2^32 float inputs and returns the order-independent checksum
 * sum_x mix64(bits(x) << 32 | bits(softplus(x))) (NaN results canonicalised).  It must equal
 * the checksum oracle/libm_sweep.c computes from the host C library.  Allocates 8 bytes.
 */
int gf_selftest_softplus(uint64_t* checksum_host, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GAUSSFIELD_H_ */
