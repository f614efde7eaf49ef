/*
 * hi3d_amd — C ABI of the MI355X (gfx950) sparse-tensor hot path of the Hi3D refiner:
 * voxel-hash kernel maps, gather-MFMA sparse convolution (submanifold and 2x2x2/s2 with
 * its transpose), the W8A8 int8 linear and the LayerNorm+adaLN row kernel.
 *
 * Conventions
 *  - Every pointer argument named *_dev is device memory owned by the caller; host
 *    arrays are named *_host. The library never allocates: scratch comes from a
 *    caller-provided workspace whose size the matching *_workspace() call reports.
 *  - Calls are asynchronous on `stream` (a hipStream_t; NULL = default stream) and
 *    return HI3D_OK or an error code; hi3d_last_error() gives the message of the
 *    calling thread's last failure. Errors found by kernels (duplicate coordinates,
 *    hash overflow, out-of-range coordinates) are OR-ed into a caller-provided device
 *    status word, which the caller reads after the stream has reached that point.
 *  - Coordinates are int32 [N, 4] rows (batch, x, y, z), as in the reference's
 *    SparseConvTensor.indices (src/hi3d_mac/torch_backend/sparse_conv.py:78-106).
 *  - A neighbour table is int32 [N, K] with K = ksize^3 and flat kernel offset
 *    k = r0*ksize^2 + r1*ksize + r2 (x-major), entry = row of the voxel at
 *    coords[o] + r - ksize/2, or N when absent
 *    (src/hi3d_mac/mlx_backend/sparse.py:20-43).
 *  - Weights use spconv's layout [Cout, K, Cin]
 *    (src/hi3d_mac/torch_backend/sparse_conv.py:230).
 */
#ifndef HI3D_AMD_H
#define HI3D_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum hi3d_status {
  HI3D_OK = 0,
  HI3D_ERR_INVALID = 1,   /* bad argument (shape, dtype, null pointer, small workspace) */
  HI3D_ERR_HIP = 2,       /* a HIP runtime call or kernel launch failed */
  HI3D_ERR_UNSUPPORTED = 3
};

/* Bits of the device status word written by map-building kernels. */
enum hi3d_map_flags {
  HI3D_MAP_DUPLICATE = 1, /* two rows share a coordinate */
  HI3D_MAP_OVERFLOW = 2,  /* the hash table ran out of free slots */
  HI3D_MAP_RANGE = 4      /* a coordinate lies outside [0, spatial_shape) or the batch */
};

enum hi3d_dtype { HI3D_F32 = 0, HI3D_F16 = 1, HI3D_BF16 = 2, HI3D_F64 = 3, HI3D_I32 = 4, HI3D_I64 = 5 };

enum hi3d_act { HI3D_ACT_NONE = 0, HI3D_ACT_SILU = 1 };

/* Message of the calling thread's last failed call ("" if none). */
const char* hi3d_last_error(void);

/* Library version string. */
const char* hi3d_version(void);

/* ------------------------------------------------------------------ kernel maps -- */

/* Workspace bytes of hi3d_kmap_subm for n voxels: the brick hash of `capacity` buckets
 * (a power of two; 0 = default, the power of two >= n) plus the cell-order sort. key64 is
 * accepted for the ABI's sake and ignored (brick keys are 64-bit). */
int hi3d_kmap_workspace(int64_t n, int64_t capacity, int32_t key64, int64_t* bytes_host);

/* Submanifold kernel map through a brick hash: the voxels of each 2x2x2 brick claim (one
 * 64-bit CAS per brick) its bucket, keyed by the brick's packed coordinates (as
 * ((b*sx + x)*sy + y)*sz + z over the halved extents, below 2^56; open addressing, the
 * home buckets of an 8x8x8-cell superblock's bricks one hashed run, double hashing past
 * it), and set their corners' bits (in the key's word) and rows; the ksize^3
 * neighbourhood of each voxel is then read bucket by bucket, writing the dense neighbour
 * table nbr_dev [n, ksize^3] (sentinel n) and per-offset non-sentinel counts counts_dev
 * [ksize^3]. Neighbours outside [0, spatial_shape) are absent. Tables above 16 MiB are
 * built and probed in superblock order. status_dev flags DUPLICATE, RANGE and OVERFLOW
 * (capacity smaller than the occupied bricks).
 * Replaces: _voxel_keys + subm_pairs (src/hi3d_mac/torch_backend/sparse_conv.py:109-149)
 * and neighbour_table (src/hi3d_mac/mlx_backend/sparse.py:29-43). */
int hi3d_kmap_subm(const int32_t* coords_dev, int64_t n, int32_t sx, int32_t sy, int32_t sz,
                   int32_t batch_size, int32_t ksize, int64_t capacity, void* workspace_dev,
                   int64_t workspace_bytes, int32_t* nbr_dev, int32_t* counts_dev,
                   int32_t* status_dev, void* stream);

/* Bytes of the device array that holds hi3d_kmap_subm_noalloc's hash table (one copy
 * per GPU the library runs on, held until the process ends). */
#define HI3D_KMAP_NOALLOC_BYTES (128ll << 20)

/* hi3d_kmap_subm without allocation or workspace: the same table, counts and status
 * (identical for every coordinate set), through a voxel-slot hash (one 64-bit slot per
 * voxel, 2n slots, each voxel's home slot its corner in an 8-slot run of its 2x2x2
 * brick) in a fixed device array of HI3D_KMAP_NOALLOC_BYTES. No counterpart in the reference: for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). Takes up to 2^23 voxels with 32-bit keys and 2^22 with 64-bit
 * keys (batch*sx*sy*sz >= 2^32 - 1); larger sets return HI3D_ERR_INVALID before any
 * launch. Every call on a GPU reuses that GPU's array, so calls that overlap on one GPU
 * (two streams or two host threads) race. */
int hi3d_kmap_subm_noalloc(const int32_t* coords_dev, int64_t n, int32_t sx, int32_t sy, int32_t sz,
                           int32_t batch_size, int32_t ksize, int32_t* nbr_dev, int32_t* counts_dev,
                           int32_t* status_dev, void* stream);

/* Workspace bytes of hi3d_kmap_subm_dense: one int32 cell per grid position
 * (batch_size*sx*sy*sz <= 2^31) and 16 pad cells before and after the grid. */
int hi3d_kmap_dense_workspace(int32_t batch_size, int32_t sx, int32_t sy, int32_t sz, int64_t* bytes_host);

/* The submanifold kernel map of hi3d_kmap_subm (same table, counts and status flags;
 * HI3D_MAP_OVERFLOW never set) through a dense grid of rows instead of the hash: for
 * grids small enough to clear, the lookups of neighbouring rows read neighbouring
 * cells. Replaces the dense-grid lookup of neighbour_table
 * (src/hi3d_mac/mlx_backend/sparse.py:29-43). */
int hi3d_kmap_subm_dense(const int32_t* coords_dev, int64_t n, int32_t sx, int32_t sy, int32_t sz,
                         int32_t batch_size, int32_t ksize, void* workspace_dev, int64_t workspace_bytes,
                         int32_t* nbr_dev, int32_t* counts_dev, int32_t* status_dev, void* stream);

/* Workspace bytes of the row ordering of hi3d_kmap_subm_dense_kept for n voxels (cell
 * keys, row ids and a radix sort). */
int hi3d_kmap_dense_order_workspace(int64_t n, int64_t* bytes_host);

/* hi3d_kmap_subm_dense over a grid that persists between calls: grid_dev (its size
 * from hi3d_kmap_dense_workspace) holds -1 in every cell on entry and is left so on
 * return (the cells the rows claim are put back after the lookup), so a call costs
 * O(n) instead of clearing 4 bytes per grid cell (4 GiB at 1024^3). The caller fills a
 * new grid with -1 once; calls sharing a grid must not overlap. order_dev (NULL, or
 * hi3d_kmap_dense_order_workspace bytes) makes the store, lookup and restore visit the
 * rows sorted by the top 16 bits of their cell keys, so neighbouring rows read
 * neighbouring cells whatever the input order; the table, counts and flags are the same
 * either way. Same reference interface as hi3d_kmap_subm_dense. */
int hi3d_kmap_subm_dense_kept(const int32_t* coords_dev, int64_t n, int32_t sx, int32_t sy, int32_t sz,
                              int32_t batch_size, int32_t ksize, void* grid_dev, int64_t grid_bytes, void* order_dev,
                              int64_t order_bytes, int32_t* nbr_dev, int32_t* counts_dev, int32_t* status_dev,
                              void* stream);

/* Workspace bytes of hi3d_kmap_pairs. */
int hi3d_kmap_pairs_workspace(int64_t n, int32_t kvol, int64_t* bytes_host);

/* Per-offset pair lists in spconv's orientation: for offset k the pairs
 * (i, nbr[i, kvol-1-k]) of every row i (ascending) whose entry is present, written
 * back to back: list k occupies [offsets[k], offsets[k+1]) of src_dev/dst_dev.
 * offsets_dev [kvol+1] is int64. An input at coords[src] feeds the output at
 * coords[dst] = coords[src] + ksize/2 - r_k.
 * Replaces: subm_pairs' (sources, targets) lists and _PairTable / get_indice_pairs
 * (src/hi3d_mac/torch_backend/sparse_conv.py:37-50,115-149,264-283). */
int hi3d_kmap_pairs(const int32_t* nbr_dev, int64_t n, int32_t kvol, void* workspace_dev,
                    int64_t workspace_bytes, int32_t* src_dev, int32_t* dst_dev,
                    int64_t* offsets_dev, void* stream);

/* Workspace bytes of hi3d_downsample_structure. */
int hi3d_downsample_workspace(int64_t n, int64_t* bytes_host);

/* 2x2x2 / stride-2 coarse structure: low = sorted unique (b, x>>1, y>>1, z>>1)
 * (lexicographic), inverse[i] = coarse row of fine row i, counts[c] = children of c,
 * slot[i] = (x&1)*4 + (y&1)*2 + (z&1). n_low_dev receives the coarse row count (int64).
 * low_dev must hold n rows of 4 int32 (only the first n_low are written); counts_dev n.
 * status_dev (one int32, may be NULL) is cleared, then receives HI3D_MAP_RANGE for a
 * coordinate outside [0, batch_size) x [0, sx) x [0, sy) x [0, sz) and
 * HI3D_MAP_DUPLICATE for a repeated coordinate; the outputs are then meaningless.
 * Replaces: downsample_structure (src/hi3d_mac/mlx_backend/sparse.py:217-233) and the
 * coordinate part of SparseDownsample (src/sparc3d/nn/sparse/spatial.py:34-63). */
int hi3d_downsample_structure(const int32_t* coords_dev, int64_t n, int32_t sx, int32_t sy,
                              int32_t sz, int32_t batch_size, void* workspace_dev,
                              int64_t workspace_bytes, int32_t* low_dev, int32_t* inverse_dev,
                              int32_t* counts_dev, uint8_t* slot_dev, int64_t* n_low_dev,
                              int32_t* status_dev, void* stream);

/* Gather tables of the strided pair: down_dev [n_low, 8] = fine row of child slot s of
 * each coarse voxel (sentinel n), up_dev [n, 8] = coarse parent in column slot[i] and
 * n_low elsewhere. Either output may be NULL.
 * (No reference function: the reference raises for stride != 1,
 * src/sparc3d/ops/sparse_backend.py:184-191; the slot order follows
 * src/hi3d_mac/mlx_backend/sparse.py:46-61.) */
int hi3d_stride2_tables(const int32_t* inverse_dev, const uint8_t* slot_dev, int64_t n,
                        int64_t n_low, int32_t* down_dev, int32_t* up_dev, void* stream);

/* The coarse structure of a downsampling by (fx, fy, fz) per axis (fx fy fz <= 256), as
 * hi3d_downsample_structure (which is this with factor 2, 2, 2; same workspace): coarse
 * coordinates (b, x / fx, y / fy, z / fz) in lexicographic order, inverse, counts, and
 * each fine row's slot ((x % fx) fy + y % fy) fz + z % fz.
 * Replaces: SparseDownsample's unique of the divided coordinates
 * (src/sparc3d/nn/sparse/spatial.py:36-50,64-72). */
int hi3d_resample_structure(const int32_t* coords_dev, int64_t n, int32_t sx, int32_t sy, int32_t sz,
                            int32_t batch_size, int32_t fx, int32_t fy, int32_t fz, void* workspace_dev,
                            int64_t workspace_bytes, int32_t* low_dev, int32_t* inverse_dev,
                            int32_t* counts_dev, uint8_t* slot_dev, int64_t* n_low_dev,
                            int32_t* status_dev, void* stream);

/* down_dev [n_low, slots]: the fine row in each slot of each coarse cell (sentinel n),
 * from hi3d_resample_structure's inverse and slot; the gather table of the mean pool
 * (hi3d_gather_mean with kvol = slots, extra = 1).
 * Replaces: SparseDownsample's scatter_reduce(mean) index
 * (src/sparc3d/nn/sparse/spatial.py:51-62). */
int hi3d_resample_down_table(const int32_t* inverse_dev, const uint8_t* slot_dev, int64_t n, int64_t n_low,
                             int32_t slots, int32_t* down_dev, void* stream);

/* Whether hi3d_stride2_up_conv takes this shape (1) or not (0): F16 / BF16, cin 64 or
 * 128, cout 64. */
int hi3d_stride2_up_supported(int32_t cin, int32_t cout, int32_t dtype);

/* Transpose of the strided convolution onto the fine set, parent-major:
 * out[down[c, s]] = bias + W[:, s, :] in[c] for every coarse row c and slot s with
 * down[c, s] < n_f. in_dev [n_c, cin], weight_dev [cout, 8, cin] (spconv's
 * [cout, 2, 2, 2, cin]), bias_dev [cout] or NULL, down_dev the [n_c, 8] table of
 * hi3d_stride2_tables, out_dev [n_f, cout]; every fine row has exactly one (parent,
 * slot), so every output row is written once. fp32 accumulation, bias added in fp32,
 * one rounding. 16-byte aligned in, weight and out; n_f * cout * 2 < 2^31.
 * (No reference function, as for hi3d_stride2_tables: the strided pair's up half,
 * SparseInverseConv3d over the spconv weight layout of
 * src/sparc3d/nn/sparse/conv.py:27-35.) */
int hi3d_stride2_up_conv(const void* in_dev, int64_t n_c, int32_t cin, const void* weight_dev,
                         const void* bias_dev, int32_t cout, const int32_t* down_dev, int64_t n_f,
                         int32_t dtype, void* out_dev, void* stream);

/* Coarse rows per tile of the parent-major up convolution (32): the sorted form's
 * order and child table hold whole tiles, ceil(n_c / 32) * 32 rows. */
int hi3d_stride2_up_tile_rows(void);

/* Workspace bytes of hi3d_stride2_up_plan. */
int hi3d_stride2_up_plan_workspace(int64_t n_c, int64_t* bytes_host);

/* Plan of the sorted up convolution: a stable radix sort of the coarse rows by
 * (row >> window_log2, 8-bit mask of the slots holding a child), so the rows of a tile
 * mostly share one mask. order_dev [ceil(n_c/32)*32] receives the coarse row of each
 * position (padding: n_c - 1), down_sorted_dev [same, 8] the permuted rows of down_dev
 * (padding: every slot n_f). window_log2 = 31 sorts all rows as one window.
 * (No reference function, as for hi3d_stride2_up_conv.) */
int hi3d_stride2_up_plan(const int32_t* down_dev, int64_t n_c, int64_t n_f, int32_t window_log2,
                         void* workspace_dev, int64_t workspace_bytes, int32_t* order_dev,
                         int32_t* down_sorted_dev, void* stream);

/* hi3d_stride2_up_conv over the plan's order: the tile at positions 32 t .. 32 t + 31
 * reads coarse rows order_dev[...] and writes the children of down_sorted_dev; a slot no
 * row of a tile has skips its products. The same outputs as hi3d_stride2_up_conv, bit
 * for bit. (No reference function, as for hi3d_stride2_up_conv.) */
int hi3d_stride2_up_conv_sorted(const void* in_dev, int64_t n_c, int32_t cin, const void* weight_dev,
                                const void* bias_dev, int32_t cout, const int32_t* order_dev,
                                const int32_t* down_sorted_dev, int64_t n_f, int32_t dtype,
                                void* out_dev, void* stream);

/* Workspace bytes of hi3d_child_neighbour_table. */
int hi3d_child_table_workspace(int64_t n_parents, int64_t* bytes_host);

/* Octree children's neighbour table from the parent table [P, 27] (sentinel P) and the
 * child occupancy mask [P, 8] (uint8 0/1), without hashing: child c = (parent p, slot s)
 * in parent-major, slot-minor order; table_dev [C, 27] (sentinel C), parent_dev [C],
 * slot_dev [C]. Buffers hold P*8 rows; n_children_dev receives C (int64).
 * Replaces: child_neighbour_table / _child_offset_tables
 * (src/hi3d_mac/mlx_backend/sparse.py:46-95). */
int hi3d_child_neighbour_table(const int32_t* parent_table_dev, const uint8_t* mask_dev,
                               int64_t n_parents, void* workspace_dev, int64_t workspace_bytes,
                               int32_t* table_dev, int32_t* parent_dev, int32_t* slot_dev,
                               int64_t* n_children_dev, void* stream);

/* ------------------------------------------------------------ convolution plans -- */

/* Rows per tile of the gather-MFMA convolution. */
int32_t hi3d_conv_tile_rows(void);

/* Workspace bytes of hi3d_conv_plan. */
int hi3d_conv_plan_workspace(int64_t n_out, int64_t* bytes_host);

/* Execution plan of a gather convolution over table_dev [n_out, kvol] (entries >= n_in
 * are absent): output rows are ordered by Morton code of coords_dev (NULL = row
 * order), then grouped by their neighbour-presence mask within windows of
 * window_rows rows (0 = one window), and cut into tiles of hi3d_conv_tile_rows() rows.
 * coord_bits (<= 19) and batch_bits (<= 7) bound the coordinates and batch indices
 * (< 2^bits) so that the Morton sort runs over 3 * coord_bits + batch_bits key bits;
 * 0 and 0 sort the full 64-bit key. Coordinates beyond the bits still give a valid
 * plan, in a coarser order.
 * Outputs: rows_dev [ntiles*T] (output row per tile slot, -1 past n_out),
 * gidx_dev [ntiles, kvol, T] (input row per tile slot and offset, n_in if absent) and
 * tile_mask_dev [ntiles] (offsets present in the tile; kvol <= 32, else all ones).
 * Built once per coordinate set and reused by every convolution over it, like the
 * reference's indice_dict cache (src/sparc3d/ops/sparse_backend.py:52-56,124-127). */
int hi3d_conv_plan(const int32_t* table_dev, int64_t n_out, int32_t kvol, int64_t n_in,
                   const int32_t* coords_dev, int32_t coord_bits, int32_t batch_bits, int64_t window_rows,
                   void* workspace_dev, int64_t workspace_bytes, int32_t* rows_dev, int32_t* gidx_dev,
                   uint32_t* tile_mask_dev, void* stream);

/* Gather-MFMA convolution: out[o] = act(bias + sum_k in[table[o,k]] . W[:, k, :]^T)
 * (+ residual[o] after act), fp32 accumulation, every output row written once.
 * in_dev [n_in, cin], weight_dev [cout, kvol, cin], bias_dev [cout] or NULL,
 * residual_dev [n_out, cout] or NULL, out_dev [n_out, cout]; all of dtype (F32, F16,
 * BF16). Requires cin*elem % 16 == 0 and 16-byte aligned pointers.
 * Replaces: subm_conv / SubMConv3d.forward (src/hi3d_mac/torch_backend/sparse_conv.py:
 * 152-195,244-247), SubMConv3d._large_forward (src/sparc3d/ops/sparse_backend.py:47-128)
 * and sparse_conv (src/hi3d_mac/mlx_backend/sparse.py:191-214). */
int hi3d_gather_conv(const void* in_dev, int64_t n_in, int32_t cin, const void* weight_dev,
                     const void* bias_dev, int32_t cout, int32_t kvol, const int32_t* rows_dev,
                     const int32_t* gidx_dev, const uint32_t* tile_mask_dev, int64_t n_out,
                     const void* residual_dev, int32_t act, int32_t dtype, void* out_dev,
                     void* stream);

/* hi3d_gather_conv (fp16, no activation, no residual) into 128 output channels with the
 * transformer res block's second norm applied to each output row before it is stored:
 * h = conv row (fp16), then LayerNorm over its 128 channels (fp32 two-pass statistics,
 * no affine), fp16(fp16(h * scale1p[b]) + shift[b]) and the fp16 SiLU, b = the row's
 * batch (coords_dev[4 r], clamped to [0, batches)); bitwise hi3d_gather_conv followed by
 * hi3d_layer_norm_act. cin in 128..512, a multiple of 64; scale1p_dev and shift_dev
 * fp16 [batches, 128]; the same plan arguments as hi3d_gather_conv.
 * Replaces: conv1 then norm2 * (1 + scale) + shift and SiLU of SparseResBlock3d.forward
 * (src/sparc3d/models/transformers/sparc3d_transformer.py:137-141;
 * src/hi3d_mac/mlx_backend/transformer.py:418-433). */
int hi3d_gather_conv_ln_silu(const void* in_dev, int64_t n_in, int32_t cin, const void* weight_dev,
                             const void* bias_dev, int32_t cout, int32_t kvol, const int32_t* rows_dev,
                             const int32_t* gidx_dev, const uint32_t* tile_mask_dev, int64_t n_out,
                             const int32_t* coords_dev, int32_t batches, const void* scale1p_dev,
                             const void* shift_dev, float eps, void* out_dev, void* stream);

/* The same convolution straight from a table [n_out, kvol], one thread per output
 * element: any channel count and F64 as well. Used for shapes the MFMA path does not
 * take (e.g. the reference's C 5->7 float64 case, tests/test_backends.py:32-50). */
int hi3d_gather_conv_simple(const void* in_dev, int64_t n_in, int32_t cin,
                            const void* weight_dev, const void* bias_dev, int32_t cout,
                            int32_t kvol, const int32_t* table_dev, int64_t n_out,
                            const void* residual_dev, int32_t act, int32_t dtype, void* out_dev,
                            void* stream);

/* The convolution of hi3d_gather_conv over the same plan for at most 16 output
 * channels: 16x16 MFMAs over 16-row parts of the plan's tiles (F16 / BF16 rows of a
 * multiple of 128 bytes, gathered through LDS) or 64-row halves (the other rows, loaded
 * to registers), offsets none of a part's rows has skipped (tile_mask_dev is not read). F32, F16 or BF16; cout 1..16, kvol <= 32,
 * cin*elem % 64 == 0, 16-byte aligned input and weight. Replaces the occupancy head's
 * gathered GEMM (SparseClsHead Conv3d(C, 8), src/hi3d_mac/mlx_backend/vae.py:270-271
 * over conv_gn_swish :166-192; src/sparc3d/models/autoencoders/blocks.py:181-197). */
int hi3d_gather_conv_narrow(const void* in_dev, int64_t n_in, int32_t cin, const void* weight_dev,
                            const void* bias_dev, int32_t cout, int32_t kvol, const int32_t* rows_dev,
                            const int32_t* gidx_dev, const uint32_t* tile_mask_dev, int64_t n_out,
                            const void* residual_dev, int32_t act, int32_t dtype, void* out_dev,
                            void* stream);

/* out_dev [n, kvol] = inverse_dev[table_dev[o, k]] where the entry is present (< n), n_low
 * where it is absent: the map of a convolution over a fine set whose inputs are the
 * coarse parents of the fine neighbours. Replaces Geometry.up_conv_index
 * (src/hi3d_mac/mlx_backend/transformer.py:253-259), which flattens it with the offset
 * for a per-tap projection. */
int hi3d_parent_table(const int32_t* table_dev, int64_t n, int32_t kvol, const int32_t* inverse_dev,
                      int64_t n_low, int32_t* out_dev, void* stream);

/* out_dev[i] = in_dev[index_dev[i]] for rows of row_bytes (a multiple of 16; 16-byte
 * aligned pointers), zero rows for indices outside [0, n_in). Replaces
 * Geometry.upsample's take (src/hi3d_mac/mlx_backend/transformer.py:265-266). */
int hi3d_gather_rows(const void* in_dev, int64_t n_in, int32_t row_bytes, const int32_t* index_dev, int64_t n,
                     void* out_dev, void* stream);

/* ------------------------------------------------------------- sort and scan -- */

/* Workspace bytes of hi3d_sort_pairs and hi3d_scan for n elements. */
int hi3d_sort_pairs_workspace(int64_t n, int64_t* bytes_host);

/* Stable LSD radix sort (8-bit digits) of n (key, int32 value) pairs by key bits
 * [begin_bit, end_bit): keys_dev (uint32 for key_bytes 4, uint64 for 8) and vals_dev
 * hold the input, keys_alt_dev / vals_alt_dev are scratch of the same sizes; the sorted
 * pairs end in the alternate buffers when *in_alt_host is 1 (an odd number of 8-bit
 * passes), else in keys_dev / vals_dev. The sort behind the kernel-map, plan, stride-2
 * and unique builds (the reference sorts with torch.sort / torch.unique /
 * mx.argsort, src/hi3d_mac/fast_unique.py:25-56). */
int hi3d_sort_pairs(void* keys_dev, void* keys_alt_dev, int32_t* vals_dev, int32_t* vals_alt_dev, int64_t n,
                    int32_t key_bytes, int32_t begin_bit, int32_t end_bit, void* workspace_dev,
                    int64_t workspace_bytes, int32_t* in_alt_host, void* stream);

/* out_dev[i] = sum of in_dev[0 .. i) (inclusive = 0) or in_dev[0 .. i] (inclusive = 1),
 * int32; out_dev may be in_dev. Workspace from hi3d_sort_pairs_workspace. */
int hi3d_scan(const int32_t* in_dev, int32_t* out_dev, int64_t n, int32_t inclusive, void* workspace_dev,
              int64_t workspace_bytes, void* stream);

/* Workspace bytes of hi3d_unique_keys. */
int hi3d_unique_keys_workspace(int64_t n, int64_t* bytes_host);

/* Sorted unique values of keys_dev [n] int64, the inverse map and run lengths, equal to
 * np.unique(keys, return_inverse=True, return_counts=True): uniq_dev [n] (first
 * *n_unique_dev entries valid), inverse_dev [n] (int64 run of each key), counts_dev [n]
 * or NULL. key_bits = 0 takes any int64; 1..63 promises keys in [0, 2^key_bits) and sorts
 * only those bits. n < 2^31 - 1.
 * Replaces unique_keys (src/hi3d_mac/fast_unique.py:25-56). */
int hi3d_unique_keys(const int64_t* keys_dev, int64_t n, int32_t key_bits, void* workspace_dev,
                     int64_t workspace_bytes, int64_t* uniq_dev, int64_t* inverse_dev, int64_t* counts_dev,
                     int64_t* n_unique_dev, void* stream);

/* Column minima lo_dev [d] and maxima hi_dev [d] (int64) of rows_dev [n, d] (I32 or
 * I64, d <= 8, n >= 1): the value ranges that hi3d_pack_rows packs. Replaces the
 * a.min / a.max of _packed_keys (src/hi3d_mac/fast_unique.py:61-62). */
int hi3d_row_bounds(const void* rows_dev, int32_t dtype, int64_t n, int32_t d, int64_t* lo_dev,
                    int64_t* hi_dev, void* stream);

/* One int64 key per row of rows_dev [n, d] (I32 or I64, d <= 8) that keeps the rows'
 * lexicographic order: key = sum_j (row[j] - lo[j]) * prod_{l > j} extent[l], with lo_dev
 * and extent_dev [d] int64 on the device (the caller checks prod(extent) < 2^62).
 * Replaces _packed_keys (src/hi3d_mac/fast_unique.py:59-71). */
int hi3d_pack_rows(const void* rows_dev, int32_t dtype, int64_t n, int32_t d, const int64_t* lo_dev,
                   const int64_t* extent_dev, int64_t* keys_dev, void* stream);

/* Inverse of hi3d_pack_rows for the first *n_dev keys (at most n_max) into rows_dev
 * [*n_dev, d]. Replaces the unpacking loop of unique_rows
 * (src/hi3d_mac/fast_unique.py:74-91). */
int hi3d_unpack_rows(const int64_t* keys_dev, int64_t n_max, const int64_t* n_dev, int32_t d,
                     const int64_t* lo_dev, const int64_t* extent_dev, void* rows_dev, int32_t dtype,
                     void* stream);

/* Mean of the present rows per table row: out[o] = sum_k in[table[o,k]] / (count + extra)
 * over entries < n_in; fp32 (F64: fp64) accumulation. With the stride-2 down table and
 * extra = 1 this is SparseDownsample's scatter_reduce(mean) onto a zero-initialised
 * output, which counts the zero as one more element
 * (src/sparc3d/nn/sparse/spatial.py:53-62). */
int hi3d_gather_mean(const void* in_dev, int64_t n_in, int32_t c, const int32_t* table_dev,
                     int32_t kvol, int64_t n_out, int32_t extra, int32_t dtype, void* out_dev,
                     void* stream);

/* Output rows per halo tile (256) and halo rows per tile (768, the last always absent). */
int32_t hi3d_halo_tile_rows(void);
int32_t hi3d_halo_capacity(void);

/* Workspace bytes of hi3d_halo_plan. */
int hi3d_halo_plan_workspace(int64_t n_out, int64_t* bytes_host);

/* Halo plan of a 27-offset submanifold table_dev [n_out, 27] (entries >= n_in absent):
 * output rows in Morton order of coords_dev (NULL = row order; coord_bits and batch_bits as
 * for hi3d_conv_plan), cut into tiles of
 * hi3d_halo_tile_rows() rows. Per tile: rows_dev [ntiles*256] (output row per slot, -1
 * past n_out), halo_dev [ntiles, 768] (sorted unique input rows touched by the tile,
 * n_in where unused), hcount_dev [ntiles], loff_dev [ntiles*256, 32] (halo position of
 * each (row, offset) for offsets 0..26, 0xffff if absent) and bmask_dev [ntiles*8]
 * (offsets present per 32-row block). *overflow_dev is set when a tile touches more
 * than 767 input rows (the plan is then unusable and the tile plan is used instead).
 * Same role as hi3d_conv_plan: built once per coordinate set and cached with the map
 * (src/sparc3d/ops/sparse_backend.py:52-56,124-127). */
int hi3d_halo_plan(const int32_t* table_dev, int64_t n_out, int32_t kvol, int64_t n_in,
                   const int32_t* coords_dev, int32_t coord_bits, int32_t batch_bits, void* workspace_dev,
                   int64_t workspace_bytes, int32_t* rows_dev, int32_t* halo_dev, int32_t* hcount_dev,
                   uint16_t* loff_dev, uint32_t* bmask_dev, int32_t* overflow_dev, void* stream);

/* The submanifold 3x3x3 convolution of hi3d_gather_conv over a halo plan: each tile's
 * halo is gathered into LDS once per 64-byte K step and shared by all 27 offsets. fp16
 * or bf16, cout a multiple of 128, cin*2 in 256..512 in steps of 64, 16-byte aligned
 * pointers. Same arguments and results as hi3d_gather_conv (fp32 accumulation).
 * Replaces: subm_conv / SubMConv3d.forward (src/hi3d_mac/torch_backend/sparse_conv.py:
 * 152-195,244-247) and sparse_conv (src/hi3d_mac/mlx_backend/sparse.py:191-214). */
int hi3d_halo_conv(const void* in_dev, int64_t n_in, int32_t cin, const void* weight_dev,
                   const void* bias_dev, int32_t cout, const int32_t* rows_dev,
                   const int32_t* halo_dev, const uint16_t* loff_dev, int64_t ntiles,
                   const void* residual_dev, int32_t act, int32_t dtype, void* out_dev,
                   void* stream);

/* -------------------------------------------------------------------- W8A8 -- */

/* Per-token symmetric int8 quantisation of x_dev [m, k] fp16: with signs_dev [k]
 * (fp32 +-1) each 64-column block is multiplied by the signs and rotated by the
 * orthonormal Sylvester-ordered Hadamard H64 (butterflies over column bits 0..5 in that
 * order, then x0.125); with signs_dev NULL no rotation. s = max(max|v|, 1e-8)/127,
 * q = clamp(rint(v/s), -127, 127). k % 64 == 0 when rotating.
 * Replaces: quantize_activation / _QUANT (src/hi3d_mac/mlx_backend/w8a8.py:25-58,95-102). */
int hi3d_w8a8_quantize(const void* x_dev, int64_t m, int32_t k, const float* signs_dev,
                       int8_t* q_dev, float* scale_dev, void* stream);

/* out[m, n] = fp16(((float)acc * sa[m]) * sw[n] + (float)bias[n]) with
 * acc = sum_k q[m,k]*w[n,k] in int32 (int8 MFMA); no FMA contraction in the epilogue.
 * q_dev [m,k] int8, w_dev [n,k] int8, sa [m], sw [n] fp32, bias [n] fp16 or NULL,
 * out_dev [m,n] fp16; acc_dev [m,n] int32 optional (NULL = not written).
 * Requires k % 16 == 0.
 * Replaces: _GEMM / linear (src/hi3d_mac/mlx_backend/w8a8.py:61-80,105-119). */
int hi3d_w8a8_gemm(const int8_t* q_dev, const float* sa_dev, const int8_t* w_dev,
                   const float* sw_dev, const void* bias_dev, int64_t m, int32_t n, int32_t k,
                   void* out_dev, int32_t* acc_dev, void* stream);

/* ------------------------------------------------- VAE GroupNorm + swish -- */

/* Workspace bytes of hi3d_group_stats (per-block partial column sums). */
int hi3d_group_stats_workspace(int64_t n, int32_t c, int64_t* bytes_host);

/* GroupNorm statistics of x_dev [n, c] (F16 / BF16 / F32, c % 8 == 0, c <= 2048, rows
 * 16-byte aligned) over `groups` groups of c / groups consecutive channels: per
 * channel fp32 sums of x and x^2, then per group mean = S1 / (n w + eps),
 * var = S2 / (n w + eps) - mean^2, inv = 1 / sqrt(var + eps), written per channel to
 * mean_dev / inv_dev [c] fp32 (n = 0 gives mean 0, inv 1 / sqrt(eps), as the divisor
 * n w + eps does; x_dev may then be NULL). Replaces SparconvVAEDecoderMLX.group_stats
 * (src/hi3d_mac/mlx_backend/vae.py:141-164). */
int hi3d_group_stats(const void* x_dev, int32_t dtype, int64_t n, int32_t c, int32_t groups, float eps,
                     void* workspace_dev, int64_t workspace_bytes, float* mean_dev, float* inv_dev,
                     void* stream);

/* out_dev [n, c] (out_dtype) = u * sigmoid(u) with u = ((x - mean) * inv) * weight + bias in
 * fp32 per channel (mean, inv, weight, bias fp32 [c], 16-byte aligned) and the sigmoid in
 * the reference's form e = 1 / (1 + exp(|u|)), u < 0 ? e : 1 - e. The activation that
 * conv_gn_swish applies while gathering (src/hi3d_mac/mlx_backend/vae.py:166-192,
 * kernels.py:240-258), computed once per row here: the convolution then gathers it. */
int hi3d_gn_swish(const void* x_dev, int32_t dtype, int64_t n, int32_t c, const float* mean_dev,
                  const float* inv_dev, const float* weight_dev, const float* bias_dev, void* out_dev,
                  int32_t out_dtype, void* stream);

/* The same activation gathered through a table: out_dev [entries, c] row j is the
 * activated row table_dev[j], zeros where table_dev[j] is outside [0, n); with a
 * [rows, kvol] table this is the [rows, kvol c] block of gather_group_norm_swish
 * (src/hi3d_mac/mlx_backend/kernels.py:261-296). */
int hi3d_gather_gn_swish(const void* x_dev, int32_t dtype, int64_t n, int32_t c,
                         const int32_t* table_dev, int64_t entries, const float* mean_dev,
                         const float* inv_dev, const float* weight_dev, const float* bias_dev,
                         void* out_dev, int32_t out_dtype, void* stream);

/* ---------------------------------------------------------- LayerNorm + adaLN -- */

/* Row LayerNorm of x_dev [rows, c] fp16 with fp32 two-pass statistics,
 * y = (x - mean) / sqrt(var + eps) (optionally * weight + bias, fp32 [c]),
 * h = fp16(y); with scale/shift (fp16 [c]) h = fp16(fp16(h*scale) + shift).
 * Replaces: layer_norm_modulate (src/hi3d_mac/mlx_backend/kernels.py:162-237) /
 * LayerNorm32 + modulate (src/sparc3d/nn/norm.py:12-17,
 * src/sparc3d/models/transformers/sparc3d_transformer.py:140). */
int hi3d_layer_norm_modulate(const void* x_dev, int64_t rows, int32_t c, float eps,
                             const float* weight_dev, const float* bias_dev,
                             const void* scale_dev, const void* shift_dev, void* out_dev,
                             void* stream);

/* The same LayerNorm (+ affine, + modulate) followed by SiLU on the fp16 result when
 * act = HI3D_ACT_SILU (sigmoid rounded to fp16, then the product): the res-block steps
 * norm1 -> SiLU and norm2 -> modulate -> SiLU in one pass.
 * Replaces: layer_norm32 + silu of _resblock / _resblock_tail
 * (src/hi3d_mac/mlx_backend/transformer.py:160-173,418-433); norm1/norm2 + F.silu of
 * SparseResBlock3d.forward (src/sparc3d/models/transformers/sparc3d_transformer.py:136-141). */
int hi3d_layer_norm_act(const void* x_dev, int64_t rows, int32_t c, float eps,
                        const float* weight_dev, const float* bias_dev,
                        const void* scale_dev, const void* shift_dev, int32_t act,
                        void* out_dev, void* stream);

/* The same LayerNorm (+ affine, + modulate) followed by the W8A8 activation quantiser
 * of its fp16 result, in one pass (the fp16 rows are not stored): q_dev [rows, c] int8
 * and q_scale_dev [rows] fp32, bitwise those of hi3d_layer_norm_modulate then
 * hi3d_w8a8_quantize with the same signs_dev (signed H64 when given, c % 64 == 0;
 * NULL = plain per-token). c a multiple of 8, at most 4096; x, the per-channel vectors
 * and signs 16-byte aligned, q 8-byte aligned.
 * Replaces: norm followed by w8a8.linear's quantize_activation in the transformer
 * block (src/hi3d_mac/mlx_backend/transformer.py:548-549, 570-571, 575-577 over
 * kernels.py:162-237 and w8a8.py:25-58, 95-102). */
int hi3d_layer_norm_quantize(const void* x_dev, int64_t rows, int32_t c, float eps,
                             const float* weight_dev, const float* bias_dev,
                             const void* scale_dev, const void* shift_dev,
                             const float* signs_dev, int8_t* q_dev, float* q_scale_dev,
                             void* stream);

/* Row-wise linear layer on fp16 rows: out_dev [n, cout] = fp16(x W^T + bias), then with
 * residual_dev fp16(out + residual) (the residual added to the rounded product and rounded
 * again, as the convolution epilogues do; the bits of hi3d_gather_conv over the one-offset
 * identity plan). x_dev [n, cin], w_dev [cout, cin], bias_dev [cout] or NULL, residual_dev
 * [n, cout] or NULL (may be out_dev). cin a multiple of 16 up to 128, cout 64, 128, 192
 * or 256; rows and weights 16-byte aligned.
 * Replaces: the res block's linear(h) + skip_connection(x)
 * (src/sparc3d/models/transformers/sparc3d_transformer.py:143-144;
 * src/hi3d_mac/mlx_backend/transformer.py:426-437). */
int hi3d_dense_linear(const void* x_dev, int64_t n, int32_t cin, const void* w_dev,
                      const void* bias_dev, int32_t cout, const void* residual_dev,
                      void* out_dev, void* stream);

/* adaLN projection: y = W . (silu(cond) if apply_silu else cond) + b in fp32
 * (W [n_out, n_in] fp32, cond [n_in], b [n_out] or NULL), then
 * scale1p_dev = fp16(1 + fp16(y[:n_out/2])) and shift_dev = fp16(y[n_out/2:])
 * (the chunk order (scale, shift) of _emb_scale_shift,
 * src/hi3d_mac/mlx_backend/transformer.py:413-416, and the fp16 rounding of (1 + scale),
 * src/hi3d_mac/mlx_backend/transformer.py:547-548). */
int hi3d_adaln_projection(const float* w_dev, const float* b_dev, const float* cond_dev,
                          int32_t n_out, int32_t n_in, int32_t apply_silu, void* scale1p_dev,
                          void* shift_dev, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HI3D_AMD_H */
