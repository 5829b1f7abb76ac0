// Internal types of libaclsparse_hip: handle, descriptors, SpMV workspace
// layout and the launcher interface between the host C ABI and the gfx950
// kernels.  Nothing here is part of the public ABI.
#pragma once

#include <cstddef>
#include <cstdint>

#include "cann_ops_sparse.h"

namespace aclsp {

// Opaque-object signatures.  Same values as the reference so that foreign or
// stale pointers fail the same way (sparse/common/aclsparse_handle_internal.h:28,
// sparse/common/aclsparse_descr_internal.h:87-89).
constexpr uint32_t kHandleSignature = 0xAC1F9501U;
constexpr uint32_t kSpMatSignature = 0x53504D54U;
constexpr uint32_t kDnVecSignature = 0xD0D2D4D6U;
constexpr uint32_t kSpMVOpDescrSignature = 0x534D5644U;  // "SMVD"
constexpr uint32_t kSpMVOpPlanSignature = 0x534D5650U;   // "SMVP"
constexpr uint32_t kDnMatSignature = 0xD0D2D4D8U;
constexpr uint32_t kSpMMOpDescrSignature = 0x534D4D44U;  // "SMMD"
constexpr uint32_t kSpMMOpPlanSignature = 0x534D4D50U;   // "SMMP"

constexpr int kVersion = 10000;  // 1.0.0, encoded MAJOR*10000+MINOR*100+PATCH
constexpr size_t kDefaultWorkspaceBytes = 4U * 1024U * 1024U;

// A pinned 4-byte host copy of a path flag and the event recorded after the
// copy; slots live in a process-wide pool (spmv_host.cpp) and are never freed.
struct ChoiceSlot;

}  // namespace aclsp

// The public typedefs name these structs in the global namespace.
struct aclsparseContext {
    uint32_t signature = aclsp::kHandleSignature;
    aclrtStream stream = nullptr;  // null = unset; ACL_SPARSE_HIP_NULL_STREAM = HIP null stream
    // Bumped on every stream change; a preprocess plan records it so that a
    // stream switch A->B->A cannot revive a plan made on the old epoch
    // (sparse/common/aclsparse_auxiliary.cpp:162-179).
    uint64_t stream_epoch = 0;
    aclsparsePointerMode_t pointer_mode = ACL_SPARSE_POINTER_MODE_HOST;
    void* default_workspace = nullptr;  // allocated lazily by aclsparseGetWorkspace
    size_t default_workspace_size = 0;
    void* user_workspace = nullptr;
    size_t user_workspace_size = 0;
};

// Fingerprint of the last aclsparseSpMVPreprocess on a matrix.  aclsparseSpMV
// skips the partition kernel only when every field still matches
// (sparse/spmv/arch35/spmv.h:46-109).
struct SpmvPlan {
    const void* buffer = nullptr;
    const void* row_offsets = nullptr;
    const void* col_ind = nullptr;
    const void* values = nullptr;
    int64_t row_stride = 1, col_stride = 1, val_stride = 1, x_stride = 1, y_stride = 1;
    uint64_t rows = 0, cols = 0, nnz = 0;
    aclsparseIndexBase_t base = ACL_SPARSE_INDEX_BASE_ZERO;
    aclsparseIndexType_t ptr_type = ACL_SPARSE_INDEX_32I;
    aclDataType value_type = ACL_FLOAT, x_type = ACL_FLOAT, y_type = ACL_FLOAT, compute_type = ACL_FLOAT;
    aclsparseOperation_t op = ACL_SPARSE_OP_NON_TRANSPOSE;
    int32_t alg = -1;
    aclrtStream stream = nullptr;
    uint64_t stream_epoch = 0;
    bool staged = false;  // Preprocess built the staged-gather tables in the buffer
    bool narrow = false;  // Preprocess built the narrow column copy (if every entry fits)
    bool cband = false;   // Preprocess wrote the complex banded transpose's CSC rows and decision
};

struct aclsparseSpMatDescr {
    uint32_t signature = aclsp::kSpMatSignature;
    aclsparseFormat_t format = ACL_SPARSE_FORMAT_CSR;
    uint64_t rows = 0, cols = 0, nnz = 0;
    void* ptrs = nullptr;    // row offsets
    void* idxs = nullptr;    // column indices
    void* values = nullptr;
    aclsparseIndexType_t ptr_type = ACL_SPARSE_INDEX_32I;
    aclsparseIndexType_t idx_type = ACL_SPARSE_INDEX_32I;
    aclsparseIndexBase_t base = ACL_SPARSE_INDEX_BASE_ZERO;
    aclDataType value_type = ACL_FLOAT;
    int64_t ptr_stride = 1, idx_stride = 1, value_stride = 1;  // in elements
    SpmvPlan plan;  // plan.buffer == nullptr means "no active SpMV plan"
    // The path the last staged Preprocess chose, copied from the workspace
    // header into a pooled pinned host slot with an event recorded after the
    // copy: once the copy has landed, SpMV launches only the chosen kernels
    // (outside stream capture); before that, every kernel set, each reading
    // the device flag.  Taken from the pool by Preprocess, handed back (never
    // waited for) by the next Preprocess and by aclsparseDestroySpMat.
    aclsp::ChoiceSlot* staged_choice = nullptr;
};

struct aclsparseDnVecDescr {
    uint32_t signature = aclsp::kDnVecSignature;
    uint64_t nums = 0;
    void* values = nullptr;
    aclDataType value_type = ACL_FLOAT;
    int64_t stride = 1;
};

struct aclsparseDnMatDescr {
    uint32_t signature = aclsp::kDnMatSignature;
    int64_t rows = 0, cols = 0, ld = 0;
    void* values = nullptr;
    aclDataType value_type = ACL_FLOAT;
    aclsparseOrder_t order = ACL_SPARSE_ORDER_ROW;
};

namespace aclsp {

// ---------------------------------------------------------------------------
// SpMV workspace layout (all offsets 64-byte aligned):
//   [0, 192)            SpmvWsHeader, written by the preprocess kernel
//   [192, ...)          normalised row offsets: rowPtr[i*stride]-base clamped
//                       to [0, nnz], rows+1 entries of 4 (I32) or 8 (I64) bytes.
//                       Same place as the reference's normalised copy
//                       (sparse/spmv/arch35/spmv_tiling_data.h:77-79).
//   block_row_start     int32[num_blocks+1]: first row of each row block
//   block_nnz_start     RowT[num_blocks+1]: normalised offset of that row
//                       (lets a block start streaming before reading its rows)
//   sink                512 bytes the kernel stores into for lanes that have
//                       no output row this chunk (keeps stores branch-free)
//   accumulator         transpose without non-zeros: cols x accumulator element
// ---------------------------------------------------------------------------
constexpr size_t kWsAlign = 64;
constexpr size_t kWsHeaderBytes = 192;
constexpr uint32_t kWsMagic = 0x4D505348U;  // "HSPM"
constexpr size_t kSinkBytes = 512;

// Row-block partition parameters.  Row r has the partition coordinate
// kRowWeight*r + rowOffset[r] (non-decreasing).  Block b holds the rows whose
// coordinate lies in [b*T, (b+1)*T): at most ceil(T/kRowWeight) <= 127 rows
// (two per lane of a wave64) and about T - kRowWeight*rows non-zeros, so one
// wave handles one block with 8 non-zeros per lane for typical row lengths;
// a longer row simply makes its block span several wave chunks.
constexpr int64_t kChunkNnz = 512;         // non-zeros one wave reduces per chunk
constexpr int64_t kChunkTarget = 496;      // non-zeros per block the T formula aims at
constexpr int64_t kRowWeight = 16;
constexpr int64_t kMaxItemsPerBlock = 2032;  // ceil(2032/16) = 127 rows per block
constexpr int64_t kMaxRowsPerBlock = 127;

struct SpmvWsHeader {
    uint32_t magic;
    uint32_t version;
    uint64_t rows;
    uint64_t cols;
    uint64_t nnz;
    uint64_t items_per_block;
    uint64_t num_blocks;
    uint64_t rowptr_offset;
    uint64_t blocks_offset;
    uint64_t block_nnz_offset;
    uint64_t sink_offset;
    uint64_t acc_offset;
    uint32_t rowptr_bytes;
    uint32_t index_base;
    uint32_t op;
    uint32_t long_chunks;        // blocks of more chunks than this run as tasks
    uint64_t task_start_offset;  // 0 when the plan has no task table
    uint64_t task_block_offset;
    uint64_t max_tasks;
    // the path Preprocess chose (0 when the plan has no choice): 0 = row /
    // CSC kernels, 1 = staged gather or column-bucketed transpose, 2 = banded
    // one-pass transpose (fp32 or complex64), 3 = row kernels on the narrow
    // column copy, 4 = banded fp32 transpose on 16-bit copies, 5 = narrow
    // row kernels on entry-aligned blocks, 6 = banded complex64 transpose on
    // packed 16-bit offsets; the staged bucket and tile counts and where the
    // tile corners are
    uint32_t staged_flag;
    uint32_t staged_buckets;
    uint64_t staged_tiles;
    uint64_t staged_tile_row_offset;
    uint64_t staged_tile_nnz_offset;
    // narrow columns: nonzero when some entry's column is too far from its
    // row block's first row for 16 bits (set by Preprocess); complex64
    // transposes: the count of band checks that failed
    uint32_t narrow_bad;
    // narrow columns: nonzero when the entry-aligned row blocks do not fit
    // (some block of more than 127 rows, or whose rows run past its window);
    // complex64 transposes: nonzero when some entry's offsets exceed 16 bits
    uint32_t entry_bad;
    uint32_t reserved[6];
};
static_assert(sizeof(SpmvWsHeader) <= kWsHeaderBytes, "header must fit 192 bytes");

inline size_t AlignUp(size_t v) { return (v + kWsAlign - 1) & ~(kWsAlign - 1); }

inline int64_t ItemsPerBlock(uint64_t rows, uint64_t nnz)
{
    // T = target + kRowWeight * (rows a target-sized block holds), capped.
    if (nnz == 0) return kMaxItemsPerBlock;
    const uint64_t extra = (static_cast<uint64_t>(kRowWeight * kChunkTarget) * rows) / nnz;
    const uint64_t t = static_cast<uint64_t>(kChunkTarget) + extra;
    return t > static_cast<uint64_t>(kMaxItemsPerBlock) ? kMaxItemsPerBlock : static_cast<int64_t>(t);
}

inline int64_t NumBlocks(uint64_t rows, uint64_t nnz)
{
    const uint64_t t = static_cast<uint64_t>(ItemsPerBlock(rows, nnz));
    return static_cast<int64_t>((static_cast<uint64_t>(kRowWeight) * rows + nnz + t - 1) / t);
}

struct SpmvLayout {
    // CSR_ALG1: the reference-sized workspace (normalised row offsets, the
    // row-block partition, the long-block tasks; for a transpose a cols-long
    // accumulator for the atomic scatter): no staged, narrow or CSC tables
    bool lean = false;
    size_t rowptr_offset = 0;
    size_t blocks_offset = 0;
    size_t block_nnz_offset = 0;
    size_t sink_offset = 0;
    size_t acc_offset = 0;
    size_t total = 0;
    int64_t items_per_block = 0;
    int64_t num_blocks = 0;
    uint32_t rowptr_bytes = 4;
    // Transpose by columns (CSC pattern built by Preprocess): column offsets
    // colptr[cols+1] (RowT), the row of every entry in CSR order
    // entry_row[nnz] (int32) and, in column order, each entry's position in
    // the CSR arrays csc_pos[nnz] (RowT), plus the sort's temporary arrays
    // (key_a/key_b int32[nnz], val_b RowT[nnz], radix-sort storage).  At
    // execution time the products a_k * x_row(k) go to prod[nnz] (the
    // accumulator type, at most 8 bytes: it reuses key_a/key_b, which only
    // Preprocess needs).  A transpose without non-zeros has no CSC pattern:
    // y = beta*y, through the accumulator at acc_offset when y is not of the
    // accumulator type.  Transposes with nnz > INT32_MAX are rejected.
    bool csc = false;
    size_t colptr_offset = 0, entry_row_offset = 0, csc_pos_offset = 0, prod_offset = 0;
    // complex64 transposes with 32-bit offsets (nnz < 2^28): Preprocess
    // writes each CSC entry's row into val_b (free once the CSC pattern is
    // built) for the one-pass banded kernel (kCbandFlag)
    bool cband = false;
    // row-block partition of the CSC pattern (columns as rows), for the
    // column pass on the stream kernel: csc_blocks int32[Bc+1], csc_block_nnz RowT[Bc+1]
    size_t csc_blocks_offset = 0, csc_block_nnz_offset = 0;
    int64_t csc_items_per_block = 0, csc_num_blocks = 0;
    // compact entry rows for the product pass: per group of kRowGroup
    // entries in CSR order, group_row int32[G] (the row of the group's first
    // entry, or -1 when the group spans more than 255 rows: then entry_row
    // holds its rows) and row_delta uint8[G*kRowGroup] (row - group_row)
    size_t group_row_offset = 0, row_delta_offset = 0;
    int64_t row_groups = 0;
    size_t key_a_offset = 0, key_b_offset = 0, val_b_offset = 0, sort_offset = 0, sort_bytes = 0;
    // Long-block tasks (non-transpose, fp32 compute): a block of more than
    // kLongChunks chunks is split into one task per chunk.  task_start[B+1]
    // (exclusive scan of the per-block task counts; task_start[B] = total),
    // task_block[max_tasks], the partial sums of the rows crossing each task's
    // first / last slot (task_head / task_tail, float[max_tasks]), a per-block
    // arrival counter (task_cnt, uint32[B]) and the scan's temporary storage.
    bool tasks = false;
    int64_t max_tasks = 0;
    size_t task_start_offset = 0, task_block_offset = 0, task_head_offset = 0, task_tail_offset = 0;
    size_t task_cnt_offset = 0, task_scan_offset = 0, task_scan_bytes = 0;
    // Staged gather (non-transpose, fp32 compute, fp32/fp16/bf16 values; see
    // StageEligible): Preprocess cuts the matrix into merge-path tiles of
    // StageTileItems rows+entries and buckets every entry by the x segment
    // of its column (kStageSegmentBytes of x per bucket; bucket S holds
    // entries whose column is outside [0, cols)).  Sections:
    //   st_tile_row int32[T+1], st_tile_nnz int64[T+1]   merge-path tile corners
    //   st_counts / st_start_bm uint32[(S+1)*(T+1)]       per (bucket, tile)
    //                                                     entry counts and
    //                                                     their exclusive scan
    //   st_start uint32[(T+1)*(S+1)]                      the scan tile-major:
    //                                                     first slot of tile t's
    //                                                     run in bucket s
    //   st_scan                                           scan temporary storage
    //   st_perm uint16[nnz+8]   slot of each entry (CSR order) in its tile's
    //                           bucket-ordered runs
    //   st_cl uint16[P+8]       bucket order: column within the bucket (0 in
    //                           the runs' padding)
    //   st_xg V[P+8]            bucket order: the gathered x values (written
    //                           by every SpMV)
    // Every (tile, bucket) run is padded to a multiple of StageChunkSlots
    // slots (8 bytes of x), so the counts, starts and slots above are in
    // padded units; P = StageSlotCap bounds their total.
    //   st_head / st_tail float[T]  partial sums of the rows crossing tile ends
    //   st_metric uint64            distinct x lines per tile, summed
    // The header's staged_flag says which path Preprocess chose.
    bool staged = false;
    int64_t st_tiles = 0, st_parts = 0, st_part_size = 0, st_tile_items = 0;
    int32_t st_buckets = 0, st_wshift = 0, st_value_bytes = 0;
    size_t st_tile_row_offset = 0, st_tile_nnz_offset = 0, st_counts_offset = 0, st_start_bm_offset = 0;
    size_t st_start_offset = 0, st_scan_offset = 0, st_scan_bytes = 0, st_perm_offset = 0, st_cl_offset = 0;
    size_t st_xg_offset = 0, st_head_offset = 0, st_tail_offset = 0, st_metric_offset = 0;
    // Narrow columns (non-transpose, NarrowTypes): each
    // entry's column as a signed 16-bit offset from the first row of its row
    // block, nc int16[nnz+8], written by Preprocess when every entry fits
    // (the header's staged_flag then reads 3).  The row kernel then streams
    // 2 bytes per entry of column data instead of 4.  With the staged tables
    // it overlays st_cl: only one of the two paths is ever chosen.
    // The low 16 bits of the normalised row offsets, nr uint16[rows+2], go
    // with it: a row block of at most kLongChunks chunks spans fewer than
    // 65536 entries, so the row kernel reads 2 bytes per row of such blocks.
    // With it, the entry-aligned row blocks (see kEntryChunk): eb int32[E+1],
    // the first row starting at or after entry 480*t, and en RowT[E+1], its offset.
    bool narrow = false;
    size_t nc_offset = 0, nr_offset = 0;
    int64_t entry_blocks = 0;
    size_t eb_offset = 0, en_offset = 0;
};

#ifndef SPMV_LONG_CHUNKS
#define SPMV_LONG_CHUNKS 4
#endif
constexpr int64_t kLongChunks = SPMV_LONG_CHUNKS;  // blocks with more chunks than this are split into tasks

// Exclusive-scan temporary storage of the task table (implemented in spmv_kernels.hip).
size_t TaskScanTempBytes(int64_t n);

// ---------------------------------------------------------------------------
// Staged gather.  A matrix whose x does not fit an XCD's L2 and whose columns
// are scattered makes the row kernels fetch one 128-byte line per 2- or
// 4-byte x value.  The staged path instead (pass A) loads each x segment into
// one workgroup's LDS and writes the values its bucket's entries need, in
// bucket order (sequential reads and writes), then (pass B) each merge-path
// tile reads its runs of those values into LDS and sums its rows.  It is
// considered for matrices whose x is at least kStageL2XBytes with at least
// kStageMinNnz entries, and for those whose x is smaller (down to
// kStageMinXBytes: the row kernels' gathers then hit L2 more often and cost
// less) with at least kStageMinNnzSmallX entries; Preprocess measures the
// columns' spread and keeps the row kernels when x accesses are local
// (banded matrices).  Measured on MI355X, random columns, fp32 unless noted
// (row kernels -> staged, µs per SpMV after a flush): x 16 MB: 2 M entries
// 36 -> 45, 4 M 66 -> 50, 8 M 125 -> 61, 16 M 235 -> 83 (243 -> 90 in rows
// of 4); x 8 MB: 16 M 172 -> 83; x 4 MB: 4 M 35 -> 46, 8 M 59 -> 57; x 2 MB:
// 8 M 51 -> 59, 33.5 M fp16 169 -> 94.  The staged path costs about 35 µs of fixed
// latency (three dependent launches) plus about 3 µs per million entries.
// ---------------------------------------------------------------------------
// Rows + entries per merge-path tile: 8184 for fp32 staged gather, 16376
// for fp16 / bf16 staged gather and for the column-bucketed transpose (the
// larger tiles halve the per-tile run tables and lengthen the runs; fp32
// staged gather measured faster with the smaller ones).  A tile's padded
// slots stay below 65536 (uint16 slot numbers).
constexpr int64_t kStageTileItemsNarrow = 8184;
constexpr int64_t kStageTileItemsWide = 16376;
inline int64_t StageTileItems(bool transpose, uint32_t valueBytes)
{
    return !transpose && valueBytes == 4U ? kStageTileItemsNarrow : kStageTileItemsWide;
}
constexpr int64_t kStageMinNnz = int64_t{1} << 22;
constexpr int64_t kStageMinNnzSmallX = int64_t{1} << 24;
constexpr int64_t kStageMinXBytes = int64_t{1} << 20;
constexpr int64_t kStageL2XBytes = int64_t{8} << 20;
constexpr int64_t kStageSegmentBytes = 128 * 1024;  // x per bucket, staged in one workgroup's LDS
constexpr int32_t kStageMaxBuckets = 1024;  // x up to 128 MiB
constexpr int64_t kStageMinParts = 512;           // pass A workgroups (two per CU at least)
constexpr int64_t kStagePartTarget = int64_t{1} << 21;  // slots per pass A workgroup beyond that
// Staged gather decision: the staged path is chosen when the tiles' distinct
// x lines exceed this fraction of the entries (the row kernels then fetch
// about one line per entry).
constexpr int64_t kStageLinesPerEntryDen = 4;  // lines * 4 > nnz

size_t StageScanTempBytes(int64_t n);  // implemented in spmv_staged_kernels.hip

// Element bytes of x for which the staged path exists (0 = not eligible).
inline uint32_t StageValueBytes(aclDataType valueType, aclDataType computeType)
{
    if (computeType != ACL_FLOAT) return 0U;
    if (valueType == ACL_FLOAT) return 4U;
    if (valueType == ACL_FLOAT16 || valueType == ACL_BF16) return 2U;
    return 0U;
}

// Value / compute types whose row kernel can read narrow columns: fp32,
// fp16 and bf16 values with fp32 compute, int8 values with int32 compute.
inline bool NarrowTypes(aclDataType valueType, aclDataType computeType)
{
    if (computeType == ACL_FLOAT) {
        return valueType == ACL_FLOAT || valueType == ACL_FLOAT16 || valueType == ACL_BF16 || valueType == ACL_INT8;
    }
    if (computeType == ACL_COMPLEX64) return valueType == ACL_COMPLEX64 || valueType == ACL_FLOAT;
    return computeType == ACL_INT32 && valueType == ACL_INT8;
}

// Narrow columns are built for matrices of at least this many entries.
constexpr int64_t kNarrowMinNnz = int64_t{1} << 20;
constexpr int32_t kNarrowFlag = 3;  // staged_flag value of the narrow-column row kernel
// staged_flag value of the banded one-pass transpose on 16-bit copies of its
// two per-entry streams (each entry's row as an offset from its CSC block's
// first column, its CSR position as an offset from its CSC index), written
// by Preprocess into key_a and val_b when every entry fits
constexpr int32_t kBandedNarrowFlag = 4;
// Entry-aligned row blocks (staged_flag 5: the narrow-column row kernel on
// them): block t holds the rows that start in [480 t, 480 (t+1)); when every
// block has at most 127 rows and its rows end within 512 entries of 480 t,
// a wave can load its block's columns and values from 480 t on before its
// block's first row and offset are known.
constexpr int64_t kEntryChunk = 480;
constexpr int32_t kEntryFlag = 5;
// staged_flag value of the one-pass banded transpose of complex64 matrices
// (values and compute complex64): written by Preprocess when at least 15/16
// of the CSC entries lie within 2^16 positions of their CSR position and
// their row within 2^16 of their column (value and x gathers then stay
// local); otherwise the flag stays 0 (the CSC product and column passes).
constexpr int32_t kCbandFlag = 2;
// ... and, when every entry's row lies within 16 bits of its CSC block's
// first column and its CSR position within 16 bits of its CSC index, the
// same kernel on both packed into one word per entry (in val_b)
constexpr int32_t kCbandNarrowFlag = 6;
constexpr int32_t kMaxPathFlag = 6;  // largest path flag a host copy may hold
inline bool CbandTypes(aclDataType valueType, aclDataType computeType)
{
    return (valueType == ACL_COMPLEX64 && computeType == ACL_COMPLEX64) ||
           (valueType == ACL_FLOAT && computeType == ACL_COMPLEX64) ||
           (valueType == ACL_INT8 && computeType == ACL_INT32);
}

// Staged x values are moved in chunks of kStageChunkBytes: every (tile,
// bucket) run of staged slots is padded to a multiple of this many slots.
// (16-byte chunks measured 40 µs faster in pass B on c4 but 53 µs slower in
// pass A, whose runs then carry twice the padding.)
constexpr uint32_t kStageChunkBytes = 8;
inline uint64_t StageChunkSlots(uint32_t valueBytes) { return kStageChunkBytes / valueBytes; }

// Upper bound of the staged slots (entries plus run padding) of a matrix.
inline uint64_t StageSlotCap(uint64_t rows, uint64_t nnz, uint64_t buckets, uint32_t valueBytes)
{
    const uint64_t items = static_cast<uint64_t>(StageTileItems(false, valueBytes));
    const uint64_t tiles = (rows + nnz + items - 1) / items;
    return nnz + (StageChunkSlots(valueBytes) - 1U) * (buckets + 1U) * tiles;
}

inline bool StageEligible(uint64_t rows, uint64_t cols, uint64_t nnz, uint32_t valueBytes)
{
    if (valueBytes == 0U || rows == 0U) return false;
    const uint64_t xBytes = cols * valueBytes;
    if (xBytes < static_cast<uint64_t>(kStageMinXBytes) || nnz > 0xF0000000ULL) return false;
    const int64_t minNnz = xBytes < static_cast<uint64_t>(kStageL2XBytes) ? kStageMinNnzSmallX : kStageMinNnz;
    if (nnz < static_cast<uint64_t>(minNnz)) return false;
    const uint64_t w = static_cast<uint64_t>(kStageSegmentBytes) / valueBytes;
    const uint64_t buckets = (cols + w - 1) / w;
    if (buckets > static_cast<uint64_t>(kStageMaxBuckets)) return false;
    return StageSlotCap(rows, nnz, buckets, valueBytes) <= 0xF0000000ULL;  // slots are uint32
}

// ---------------------------------------------------------------------------
// Column-bucketed transpose (fp32 values and compute, unit strides).  The
// CSC column pass gathers each product from a CSR-ordered array as large as
// the matrix: one MALL line per 4-byte product.  Instead, Preprocess cuts the
// matrix into the same merge-path tiles and buckets every entry by its
// column (W columns per bucket, W chosen so that a bucket's entries fit one
// workgroup's LDS); pass 1 writes each tile's products as runs into bucket
// order, pass 2 loads one bucket's products into LDS, places them in column
// order (each entry's place, from the CSC pattern, is a Preprocess table) and
// sums every column in row order.  It reuses the staged sections: st_perm is
// each entry's slot in its tile's bucket-ordered runs, st_cl each slot's
// place within its bucket's column-ordered products.
// ---------------------------------------------------------------------------
constexpr int64_t kBtMinNnz = int64_t{1} << 20;
constexpr int32_t kBtMaxBuckets = 2048;
constexpr int64_t kBtRegionTarget = 24576;  // mean entries per bucket the width aims at
constexpr int64_t kBtRegionCap = 32768;     // entries per bucket that pass 2's LDS holds

// Columns per bucket (a power of two): about kBtRegionTarget entries each.
inline int32_t BtBucketShift(uint64_t cols, uint64_t nnz)
{
    const uint64_t target = nnz > 0 ? static_cast<uint64_t>(kBtRegionTarget) * cols / nnz : 65536U;
    int32_t shift = 6;
    while (shift < 16 && (uint64_t{2} << shift) <= target) ++shift;
    return shift;
}

inline bool BtEligible(uint64_t rows, uint64_t cols, uint64_t nnz, uint32_t valueBytes)
{
    if (valueBytes != 4U || rows == 0U || cols == 0U) return false;
    if (nnz < static_cast<uint64_t>(kBtMinNnz) || nnz > 0x7FFFFFFFULL) return false;
    const uint64_t w = uint64_t{1} << BtBucketShift(cols, nnz);
    return (cols + w - 1) / w <= static_cast<uint64_t>(kBtMaxBuckets);
}

// Radix-sort temporary storage for the CSC build (implemented in spmv_kernels.hip).
size_t CscSortTempBytes(int64_t nnz, uint32_t posBytes);

// Entries per group of the transpose's compact row table (one wave of 4 entries per lane).
constexpr int64_t kRowGroup = 256;

inline size_t AccumulatorBytes(aclDataType computeType)
{
    return computeType == ACL_INT32 ? 8U : computeType == ACL_COMPLEX64 ? 8U : 4U;
}

inline SpmvLayout ComputeLayout(uint64_t rows, uint64_t cols, uint64_t nnz, aclsparseIndexType_t ptrType,
                                aclDataType computeType, bool transpose, bool allowTasks = true,
                                uint32_t stageValueBytes = 0, bool narrowTypes = false, bool cbandTypes = false,
                                bool lean = false)
{
    SpmvLayout l;
    l.lean = lean;
    if (lean) {
        stageValueBytes = 0;
        narrowTypes = false;
        cbandTypes = false;
    }
    l.rowptr_bytes = ptrType == ACL_SPARSE_INDEX_64I ? 8U : 4U;
    l.items_per_block = ItemsPerBlock(rows, nnz);
    l.num_blocks = NumBlocks(rows, nnz);
    l.rowptr_offset = kWsHeaderBytes;
    // rows + 2 entries: one pad entry, so that row offsets can be read in pairs
    l.blocks_offset = AlignUp(l.rowptr_offset + static_cast<size_t>(rows + 2) * l.rowptr_bytes);
    l.block_nnz_offset = AlignUp(l.blocks_offset + static_cast<size_t>(l.num_blocks + 1) * sizeof(int32_t));
    l.sink_offset = AlignUp(l.block_nnz_offset + static_cast<size_t>(l.num_blocks + 1) * l.rowptr_bytes);
    l.acc_offset = l.sink_offset + kSinkBytes;
    l.total = l.acc_offset;
    if (allowTasks && !transpose && computeType == ACL_FLOAT && nnz > 0) {
        const int64_t maxTasks = static_cast<int64_t>(nnz / kChunkNnz) + l.num_blocks + 1;
        if (maxTasks < 0x7FFFFFFFLL) {
            l.tasks = true;
            l.max_tasks = maxTasks;
            const size_t mt = static_cast<size_t>(maxTasks);
            const size_t nb1 = static_cast<size_t>(l.num_blocks + 1);
            l.task_start_offset = AlignUp(l.total);
            l.task_block_offset = AlignUp(l.task_start_offset + nb1 * sizeof(int32_t));
            l.task_head_offset = AlignUp(l.task_block_offset + mt * sizeof(int32_t));
            l.task_tail_offset = AlignUp(l.task_head_offset + mt * sizeof(float));
            l.task_cnt_offset = AlignUp(l.task_tail_offset + mt * sizeof(float));
            l.task_scan_offset = AlignUp(l.task_cnt_offset + nb1 * sizeof(uint32_t));
            l.task_scan_bytes = TaskScanTempBytes(l.num_blocks + 1);
            l.total = AlignUp(l.task_scan_offset + l.task_scan_bytes + 256);  // re-aligned to 256 bytes at use
        }
    }
    if (transpose && lean) {
        l.total = AlignUp(l.acc_offset + static_cast<size_t>(cols) * AccumulatorBytes(computeType));
    } else if (transpose) {
        l.csc = nnz > 0 && nnz <= 0x7FFFFFFFULL;
        if (!l.csc) {
            l.total = AlignUp(l.acc_offset + static_cast<size_t>(cols) * AccumulatorBytes(computeType));
        } else {
            const size_t n = static_cast<size_t>(nnz);
            const size_t rb = l.rowptr_bytes;
            l.colptr_offset = AlignUp(l.acc_offset);
            // cols + 2 entries: a pad entry, as for the row offsets
            l.entry_row_offset = AlignUp(l.colptr_offset + static_cast<size_t>(cols + 2) * rb);
            l.csc_pos_offset = AlignUp(l.entry_row_offset + n * sizeof(int32_t));
            l.key_a_offset = AlignUp(l.csc_pos_offset + n * rb);
            l.key_b_offset = AlignUp(l.key_a_offset + n * sizeof(int32_t));
            l.val_b_offset = AlignUp(l.key_b_offset + n * sizeof(int32_t));
            l.prod_offset = l.key_a_offset;  // prod[nnz] of <= 8 bytes ends before val_b
            l.sort_offset = AlignUp(l.val_b_offset + n * rb);
            l.sort_bytes = CscSortTempBytes(static_cast<int64_t>(nnz), l.rowptr_bytes);
            l.csc_items_per_block = ItemsPerBlock(cols, nnz);
            l.csc_num_blocks = NumBlocks(cols, nnz);
            l.csc_blocks_offset = AlignUp(l.sort_offset + l.sort_bytes + 256);  // sort temp re-aligned to 256 at use
            l.csc_block_nnz_offset =
                AlignUp(l.csc_blocks_offset + static_cast<size_t>(l.csc_num_blocks + 1) * sizeof(int32_t));
            l.row_groups = static_cast<int64_t>((n + kRowGroup - 1) / kRowGroup);
            l.cband = cbandTypes && rb == 4U && nnz <= 0x0FFFFFFFULL;
            l.group_row_offset =
                AlignUp(l.csc_block_nnz_offset + static_cast<size_t>(l.csc_num_blocks + 1) * rb);
            l.row_delta_offset = AlignUp(l.group_row_offset + static_cast<size_t>(l.row_groups) * sizeof(int32_t));
            l.total = AlignUp(l.row_delta_offset + static_cast<size_t>(l.row_groups) * kRowGroup);
        }
    }
    if (transpose && l.csc && BtEligible(rows, cols, nnz, stageValueBytes)) {
        l.staged = true;
        l.st_value_bytes = 4;
        l.st_wshift = BtBucketShift(cols, nnz);
        const uint64_t w = uint64_t{1} << l.st_wshift;
        l.st_buckets = static_cast<int32_t>((cols + w - 1) / w);
        l.st_tile_items = StageTileItems(transpose, stageValueBytes);
        const uint64_t items = static_cast<uint64_t>(l.st_tile_items);
        const uint64_t t = (rows + nnz + items - 1) / items;
        l.st_tiles = static_cast<int64_t>(t);
        const size_t cells = static_cast<size_t>(l.st_buckets + 1) * static_cast<size_t>(t + 1);
        const size_t n8 = static_cast<size_t>(nnz) + 8;
        l.st_tile_row_offset = AlignUp(l.total);
        l.st_tile_nnz_offset = AlignUp(l.st_tile_row_offset + static_cast<size_t>(t + 1) * sizeof(int32_t));
        l.st_counts_offset = AlignUp(l.st_tile_nnz_offset + static_cast<size_t>(t + 1) * sizeof(int64_t));
        l.st_start_bm_offset = AlignUp(l.st_counts_offset + cells * sizeof(uint32_t));
        l.st_start_offset = AlignUp(l.st_start_bm_offset + cells * sizeof(uint32_t));
        l.st_scan_offset = AlignUp(l.st_start_offset + cells * sizeof(uint32_t));
        l.st_scan_bytes = StageScanTempBytes(static_cast<int64_t>(cells));
        l.st_perm_offset = AlignUp(l.st_scan_offset + l.st_scan_bytes + 256);  // re-aligned to 256 at use
        l.st_cl_offset = AlignUp(l.st_perm_offset + n8 * sizeof(uint16_t));
        l.st_metric_offset = AlignUp(l.st_cl_offset + n8 * sizeof(uint16_t));
        l.total = AlignUp(l.st_metric_offset + sizeof(uint64_t));
    }
    if (!transpose && StageEligible(rows, cols, nnz, stageValueBytes)) {
        l.staged = true;
        l.st_value_bytes = static_cast<int32_t>(stageValueBytes);
        const uint64_t w = static_cast<uint64_t>(kStageSegmentBytes) / stageValueBytes;
        int32_t shift = 0;
        while ((uint64_t{1} << shift) < w) ++shift;
        l.st_wshift = shift;
        l.st_buckets = static_cast<int32_t>((cols + w - 1) / w);
        l.st_tile_items = StageTileItems(transpose, stageValueBytes);
        const uint64_t items = static_cast<uint64_t>(l.st_tile_items);
        const uint64_t t = (rows + nnz + items - 1) / items;
        l.st_tiles = static_cast<int64_t>(t);
        // pass A covers the padded slots: at most slotCap (their count is
        // known on the device only; workgroups past it exit)
        // (a whole number of rounds of one workgroup per CU: 256 CUs)
        const uint64_t slotCap = StageSlotCap(rows, nnz, static_cast<uint64_t>(l.st_buckets), stageValueBytes);
        int64_t parts = static_cast<int64_t>((slotCap + kStagePartTarget - 1) / kStagePartTarget);
        parts = parts < kStageMinParts ? kStageMinParts : (parts + 255) / 256 * 256;
        int64_t part = static_cast<int64_t>((slotCap + parts - 1) / parts);
        part = (part + 7) & ~int64_t{7};
        l.st_part_size = part;
        l.st_parts = static_cast<int64_t>((slotCap + part - 1) / part);
        const size_t cells = static_cast<size_t>(l.st_buckets + 1) * static_cast<size_t>(t + 1);
        const size_t n8 = static_cast<size_t>(nnz) + 8;
        const size_t s8 = static_cast<size_t>(slotCap) + 8;
        l.st_tile_row_offset = AlignUp(l.total);
        l.st_tile_nnz_offset = AlignUp(l.st_tile_row_offset + static_cast<size_t>(t + 1) * sizeof(int32_t));
        l.st_counts_offset = AlignUp(l.st_tile_nnz_offset + static_cast<size_t>(t + 1) * sizeof(int64_t));
        l.st_start_bm_offset = AlignUp(l.st_counts_offset + cells * sizeof(uint32_t));
        l.st_start_offset = AlignUp(l.st_start_bm_offset + cells * sizeof(uint32_t));
        l.st_scan_offset = AlignUp(l.st_start_offset + cells * sizeof(uint32_t));
        l.st_scan_bytes = StageScanTempBytes(static_cast<int64_t>(cells));
        l.st_perm_offset = AlignUp(l.st_scan_offset + l.st_scan_bytes + 256);  // re-aligned to 256 at use
        l.st_cl_offset = AlignUp(l.st_perm_offset + n8 * sizeof(uint16_t));
        l.st_xg_offset = AlignUp(l.st_cl_offset + s8 * sizeof(uint16_t));
        l.st_head_offset = AlignUp(l.st_xg_offset + s8 * stageValueBytes);
        l.st_tail_offset = AlignUp(l.st_head_offset + static_cast<size_t>(t) * sizeof(float));
        l.st_metric_offset = AlignUp(l.st_tail_offset + static_cast<size_t>(t) * sizeof(float));
        l.total = AlignUp(l.st_metric_offset + sizeof(uint64_t));
    }
    if (!transpose && narrowTypes && rows > 0 && nnz >= static_cast<uint64_t>(kNarrowMinNnz)) {
        l.narrow = true;
        l.nr_offset = AlignUp(l.total);
        l.total = AlignUp(l.nr_offset + (static_cast<size_t>(rows) + 2) * sizeof(uint16_t));
        l.entry_blocks = static_cast<int64_t>((nnz + kEntryChunk - 1) / kEntryChunk);
        l.eb_offset = l.total;
        l.en_offset = AlignUp(l.eb_offset + static_cast<size_t>(l.entry_blocks + 1) * sizeof(int32_t));
        l.total = AlignUp(l.en_offset + static_cast<size_t>(l.entry_blocks + 1) * l.rowptr_bytes);
        if (l.staged) {
            l.nc_offset = l.st_cl_offset;  // st_cl holds at least nnz + 8 uint16
        } else {
            l.nc_offset = AlignUp(l.total);
            l.total = AlignUp(l.nc_offset + (static_cast<size_t>(nnz) + 8) * sizeof(int16_t));
        }
    }
    return l;
}

// Path choices made on the device by a Preprocess (spmv_host.cpp): publish
// the header's path flag to the host through a pooled pinned slot (the
// previous slot goes back to the pool), read it once the copy has completed
// (-1 before, and always under stream capture), hand the slot back.  None of
// them waits for the device.
void PublishPathChoice(ChoiceSlot*& slot, void* ws, void* stream);
int32_t QueryPathChoice(const ChoiceSlot* slot, void* stream);
void ReleasePathChoice(ChoiceSlot*& slot);

// SpMV into a workspace that scratch() returns (resolved only after the
// inputs are validated and the layout fits scratchBytes): the tables are
// rebuilt on every call and the staged path is not used (spmv_host.cpp).
aclsparseStatus_t SpmvWithScratch(aclsparseHandle_t handle, aclsparseOperation_t opA, const void* alpha,
                                  aclsparseConstSpMatDescr_t matA, aclsparseConstDnVecDescr_t vecX, const void* beta,
                                  aclsparseDnVecDescr_t vecY, aclDataType computeType, aclsparseSpMVAlg_t alg,
                                  void* (*scratch)(), size_t scratchBytes);

// ---------------------------------------------------------------------------
// Launcher interface (implemented in spmv_kernels.hip).
// ---------------------------------------------------------------------------
// UNIT: no values (every entry is 1); the transpose's column pass reads its
// fp32 products through the x gather.
// GATH: fp32 values gathered by position (the "values" array holds each
// entry's position in the caller's values): the one-pass column kernel of
// banded fp32 transposes.
enum class ValKind : int32_t { F32 = 0, F16 = 1, BF16 = 2, I8 = 3, C64 = 4, UNIT = 5, GATH = 6 };
enum class OutKind : int32_t { F32 = 0, F16 = 1, BF16 = 2, I32 = 3, C64 = 4 };
enum class AccKind : int32_t { F32 = 0, I64 = 1, C64 = 2 };

struct SpmvLaunch {
    // matrix (original descriptor pointers and strides)
    const void* row_ptr;       // original row offsets
    int64_t row_stride;
    const int32_t* col;
    int64_t col_stride;
    const void* val;
    int64_t val_stride;
    const void* x;
    int64_t x_stride;
    void* y;
    int64_t y_stride;
    int64_t rows, cols, nnz;
    int32_t base;
    int32_t rowptr64;          // 1: row offsets are int64
    ValKind val_kind;
    OutKind out_kind;
    AccKind acc_kind;
    int32_t op;                // aclsparseOperation_t
    int32_t alg;               // aclsparseSpMVAlg_t
    // scalars: host mode fills the values, device mode the pointers
    int32_t device_scalars;
    float alpha_re, alpha_im, beta_re, beta_im;
    int32_t alpha_i, beta_i;
    const void* alpha_ptr;
    const void* beta_ptr;
    // workspace
    void* ws;
    SpmvLayout layout;
    // staged gather: Preprocess builds its tables; SpMV launches its kernels
    // (which check the path flag Preprocess left in the header)
    int32_t staged;
    // narrow columns: Preprocess may have written the 16-bit column copy
    int32_t narrow;
    // complex64 transposes: Preprocess wrote each CSC entry's row and the
    // banded decision (path flag kCbandFlag)
    int32_t cband;
    // with staged, narrow or cband: the path Preprocess chose, if known on
    // the host (0 row / CSC kernels, 1 staged or column-bucketed kernels, 2
    // banded transpose kernel, 3 narrow-column row kernel), or -1: launch
    // every set, each runs only on its flag values (cband: the CSC kernels)
    int32_t staged_choice;
};

// Staged gather: tables and path decision (after LaunchSpmvPreprocess) and
// the three execution kernels (after the row kernel launched with its skip
// flag).  Implemented in spmv_staged_kernels.hip.
int LaunchStagedPreprocess(const SpmvLaunch& l, void* stream);
int LaunchStagedCompute(const SpmvLaunch& l, void* stream);

// Normalises the row offsets and writes the row-block partition and header.
int LaunchSpmvPreprocess(const SpmvLaunch& l, void* stream);
// SpMVOp on the row-block partition of l (fp32, non-transpose, no tasks):
// z = alpha*(A*x, doubly compensated) + beta*y, y read from l.y.
int LaunchSpmvOpStream(const SpmvLaunch& l, float* z, void* stream);
// The same without a partition (SpMVOp ALG1 has no buffer): blocks of a fixed
// row count taken straight from l.row_ptr (base subtracted on the fly).
int LaunchSpmvOpStreamFixed(const SpmvLaunch& l, float* z, void* stream);
// Runs y = alpha*op(A)*x + beta*y using the partition already in the workspace.
int LaunchSpmvCompute(const SpmvLaunch& l, void* stream);

}  // namespace aclsp

// ---------------------------------------------------------------------------
// SpMVOp (Z = alpha*A*X + beta*Y with a compensated dot product).
// ---------------------------------------------------------------------------
struct aclsparseSpMVOpDescr {
    uint32_t signature = aclsp::kSpMVOpDescrSignature;
    uint64_t m = 0, n = 0, nnz = 0;
    aclsparseIndexBase_t base = ACL_SPARSE_INDEX_BASE_ZERO;
    aclsparseIndexType_t row_type = ACL_SPARSE_INDEX_32I;
    const void* row_offsets = nullptr;
    const int32_t* col_ind = nullptr;
    const float* values = nullptr;
    aclsparseSpMVOpAlg_t alg = ACL_SPARSE_SPMVOP_ALG1;
    void* buffer = nullptr;   // ALG2 reorder / bin_edge tables (caller-owned)
    uint32_t num_bins = 0;    // ALG2 bins (workgroups)
    // ALG2: createDescr built the narrow column copy in the buffer; the path it
    // chose on the device, copied to pinned host memory behind an event
    bool narrow = false;
    aclsp::ChoiceSlot* choice = nullptr;
};

struct aclsparseSpMVOpPlan {
    uint32_t signature = aclsp::kSpMVOpPlanSignature;
    aclsparseSpMVOpDescr* descr = nullptr;  // weak: the descriptor must outlive the plan
    aclsparseSpMVOpAlg_t alg = ACL_SPARSE_SPMVOP_ALG1;
};

namespace aclsp {

// ALG2 workspace: the reference's fixed part (sparse/spmv_op/arch35/spmv_op.h:65-86):
//   [0,256) header | reorder[m] | tmpReorder[m] | scratch[m] | tmpScratch[m] |
//   binEdge[bins+1], every array 64-byte aligned, followed by this build's
//   extension: running[m] (int64 inclusive sums of the sorted row lengths) and
//   the device sort/scan temporary storage.
constexpr size_t kOpHeaderBytes = 256;
constexpr uint32_t kOpRowsPerBin = 128;

//   After them: the row-block partition of the execution kernel (an SpMV
//   workspace without long-block tasks, `spmv` bytes in, laid out by `sl`).
struct SpmvOpLayout {
    size_t reorder = 0, tmp_reorder = 0, scratch = 0, tmp_scratch = 0, bin_edge = 0;
    size_t running = 0, temp = 0, temp_bytes = 0, spmv = 0, total = 0;
    SpmvLayout sl;
};

// numBins = min(CUs, ceil(m/128)) (sparse/spmv_op/arch35/spmv_op_host.cpp:305-327 with
// the AIV core count replaced by the CU count).
uint32_t SpmvOpNumBins(int64_t m);
SpmvOpLayout SpmvOpComputeLayout(int64_t m, int64_t n, int64_t nnz, aclsparseIndexType_t rowType, uint32_t bins);

int LaunchSpmvOpPreprocess(const aclsparseSpMVOpDescr& d, void* stream);
// ALG2: whether createDescr builds the narrow column copy; where the SpMV
// workspace (whose header holds the path flag) starts in the buffer.
bool SpmvOpNarrowUsable(const aclsparseSpMVOpDescr& d);
void* SpmvOpSpmvWorkspace(const aclsparseSpMVOpDescr& d);
int LaunchSpmvOpExecute(const aclsparseSpMVOpDescr& d, const void* x, const void* y, void* z, float alpha,
                        float beta, const void* alphaPtr, const void* betaPtr, bool deviceScalars, void* stream);


// ---------------------------------------------------------------------------
// SpMMOp: C = alpha*A*op(B) + beta*C, A CSR (fp32 or fp16, I32/I64 row
// offsets), B and C dense in either order, fp32 accumulation.
// ---------------------------------------------------------------------------
// ALG2 workspace: the reference's part (sparse/spmm_op/arch35/spmm_op.h:63-81):
//   [0,256) header | reorder[m] | bin_edge[bins+1], 64-byte aligned,
// followed by this build's extension for the device-side table build:
//   tmp_reorder[m] | lengths[m] | sorted lengths[m] | running[m] (int64) |
//   sort/scan temporary storage.
struct SpmmOpLayout {
    size_t reorder = 0, bin_edge = 0, ref_total = 0;
    size_t tmp_reorder = 0, scratch = 0, tmp_scratch = 0, running = 0, temp = 0, temp_bytes = 0, total = 0;
};
SpmmOpLayout SpmmOpComputeLayout(int64_t m, uint32_t bins);

// Length-sorted row tables shared by SpMVOp and SpMMOp ALG2: reorder = rows
// by length, descending, stable; binEdge[0..bins] splits the sorted rows into
// bins of about ceil(total/bins) non-zeros, one edge per row at most.
struct LengthTables {
    const void* row_offsets;
    bool rowptr64;
    int64_t m;
    uint32_t bins;
    int32_t *reorder, *tmp_reorder, *scratch, *tmp_scratch, *bin_edge;
    int64_t* running;
    void* temp;
    size_t temp_bytes;
};
int LaunchLengthTables(const LengthTables& t, void* stream);

struct SpmmLaunch {
    const void* row_offsets;
    const int32_t* col_ind;
    const void* values;
    const void* b;
    void* c;
    int64_t m, k, n, ldb, ldc;
    int32_t base;
    int32_t rowptr64;
    int32_t fp16;
    int32_t high_precision;  // Kahan-compensated sums (fp32 only)
    int32_t b_trans;         // opB = T
    int32_t b_row_major, c_row_major;
    int64_t nnz;
    float alpha, beta;
    const float* alpha_ptr;  // device pointer mode: read on the device
    const float* beta_ptr;
};
int LaunchSpmmOp(const SpmmLaunch& l, void* stream);

}  // namespace aclsp

struct aclsparseSpMMOpDescr {
    uint32_t signature = aclsp::kSpMMOpDescrSignature;
    uint64_t m = 0, k = 0, nnz = 0;
    aclsparseIndexBase_t base = ACL_SPARSE_INDEX_BASE_ZERO;
    aclsparseIndexType_t row_type = ACL_SPARSE_INDEX_32I;
    aclDataType value_type = ACL_FLOAT;
    aclsparseOperation_t op_b = ACL_SPARSE_OP_NON_TRANSPOSE;
    const void* row_offsets = nullptr;
    const int32_t* col_ind = nullptr;
    const void* values = nullptr;
    aclsparseSpMMOpAlg_t alg = ACL_SPARSE_SPMMOP_ALG1;
    void* buffer = nullptr;  // ALG2 tables (caller-owned)
    uint32_t num_bins = 0;
};

struct aclsparseSpMMOpPlan {
    uint32_t signature = aclsp::kSpMMOpPlanSignature;
    aclsparseSpMMOpDescr* descr = nullptr;  // weak: the descriptor must outlive the plan
    aclsparseSpMMOpAlg_t alg = ACL_SPARSE_SPMMOP_ALG1;
};
