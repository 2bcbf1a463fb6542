/*
 * emrs.h - C ABI of the reshard-repack copy-plan executor for MI355X (gfx950).
 *
 * The reference moves optimizer state with a Python executor that slices
 * per-parameter tensors and exchanges them over injectable send/recv/broadcast
 * callables:
 *   TransferManager(send_fn, recv_fn, broadcast_fn)
 *       elastic_megatron/transfer/transfer.py:23-34
 *   TransferManager.transfer_optimizer_tensors(virtual_param_space)
 *       elastic_megatron/transfer/transfer.py:291-341
 *   TransferManager._send_optimizer_tensors / _recv_optimizer_tensors
 *       elastic_megatron/transfer/transfer.py:36-101
 *   TransferManager.redundant_backup (Group-ZeRO replication)
 *       elastic_megatron/transfer/transfer.py:343-388
 *   Communicator.send / recv (self-copy FIFO, pack/unpack copies)
 *       elastic_megatron/transfer/communicator.py:61-96
 *
 * Here the whole transfer is one precomputed plan of copy segments executed
 * by one copy kernel launch over device-resident buffers.  Every segment copies
 * `rows` rows of `len` elements of `elem_bytes` bytes each, bit for bit:
 *
 *   for r in [0, rows):
 *     dst[dst_buf][dst_off + r*dst_stride + i] = src[src_buf][src_off + r*src_stride + i],
 *     i in [0, len)
 *
 * Conventions
 *   - All offsets, lengths and strides are in elements of the segment's
 *     elem_bytes (1, 2, 4 or 8).  Mixed element sizes may share one plan.
 *   - Buffers are caller-owned device allocations; the library never
 *     allocates or frees caller memory.  A plan owns only its own tables in
 *     device memory: the segment table, the chunk table (emrs_tuning.chunk_index)
 *     and, beyond 128 buffers a side, its pointer tables.
 *   - Every function returns EMRS_OK (0) or a negative EMRS_ERR_* code and
 *     never throws across the ABI; emrs_last_error() returns a description
 *     of the last failure on the calling thread.
 *   - Work is enqueued on the caller's stream (a hipStream_t passed as
 *     void*; NULL is the null stream).  Execution is asynchronous.
 *   - A plan may be executed and compared from several threads and on
 *     several streams at once: its per-device tables are made, and the
 *     launch records emrs_plan_destroy waits on are kept, under the plan's
 *     own lock.  emrs_plan_destroy must not overlap other calls on the same
 *     plan.
 */
#ifndef EMRS_H
#define EMRS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EMRS_ABI_VERSION 8

#define EMRS_OK 0
#define EMRS_ERR_INVALID_ARGUMENT (-1)
#define EMRS_ERR_OUT_OF_BOUNDS (-2)
#define EMRS_ERR_MISALIGNED (-3)
#define EMRS_ERR_OVERLAP (-4)
#define EMRS_ERR_HIP (-5)
#define EMRS_ERR_NO_DEVICE (-6)
#define EMRS_ERR_TOO_MANY_BUFFERS (-7)
#define EMRS_ERR_ALIAS (-8)
#define EMRS_ERR_CAPTURE (-9) /* the call would allocate or upload while its stream captures a graph */
#define EMRS_ERR_TOO_LARGE (-10) /* more than the static scratch of emrs_plan_compare_static, or a shared
                                    allocation of 2 GiB or more (emrs_ipc_*) */

/* Maximum number of source (and, separately, destination) buffers.  Up to
 * 128 per side travel in kernel arguments; a plan with more on either side
 * passes its base pointers through a device table.  The plan keeps, per
 * device, the table of its first call, and its segment table resolved against
 * those pointers, and reuses both while the base pointers repeat; a call with
 * other pointers uploads a pointer table of its own and frees it on its
 * stream (hipMallocAsync / hipFreeAsync). */
#define EMRS_MAX_BUFFERS 65535

/* emrs_plan_create flags */
#define EMRS_PLAN_CHECK_DISJOINT 1u /* reject plans whose destination ranges overlap */

/* emrs_segment flags */
#define EMRS_SEG_CAST_BF16 1u /* fp32 segment that also writes its values as bf16 to aux */
#define EMRS_SEG_ZERO_FILL 2u /* write zeros instead of copying: the source is not read */
#define EMRS_SEG_DUP 4u       /* also write the values, unchanged, to aux (a second destination) */

/* One strided copy.  Units: elements of elem_bytes bytes. */
typedef struct emrs_segment {
  uint32_t src_buf;    /* index into the src_bases passed at execution */
  uint32_t dst_buf;    /* index into the dst_bases passed at execution */
  uint32_t elem_bytes; /* 1, 2, 4 or 8 */
  uint32_t flags;      /* EMRS_SEG_* bits; CAST_BF16 and DUP exclude each other */
  uint64_t src_off;    /* first element of row 0 in the source buffer */
  uint64_t dst_off;    /* first element of row 0 in the destination buffer */
  uint64_t len;        /* elements per row */
  uint64_t rows;       /* number of rows (>= 1) */
  uint64_t src_stride; /* elements between source row starts (rows > 1) */
  uint64_t dst_stride; /* elements between destination row starts (rows > 1), >= len */
  /* EMRS_SEG_CAST_BF16 (elem_bytes 4 only): every copied fp32 value is also
   * written, rounded to bf16 to nearest-even (NaN -> 0x7FC0, the rounding of
   * torch's float -> bfloat16 conversion), at bf16 element
   * aux_off + r*aux_stride + i of destination buffer aux_buf.  This is
   * Megatron's copy of main params into the bf16 model params
   * (training_state.py:176-197) fused into the reshard.
   * EMRS_SEG_DUP: every value is also written unchanged (elem_bytes wide) at
   * element aux_off + r*aux_stride + i of destination buffer aux_buf: one
   * read feeding two destinations, as a Group-ZeRO scale-up needs to fill
   * two optimizer instances from one source shard (transfer.py:343-388). */
  uint32_t aux_buf;
  uint32_t reserved;   /* must be 0 */
  uint64_t aux_off;
  uint64_t aux_stride; /* aux elements between aux row starts (rows > 1), >= len */
} emrs_segment;

typedef struct emrs_plan emrs_plan;

typedef struct emrs_plan_stats {
  uint64_t n_segments;      /* segments as given */
  uint64_t n_device_segments; /* after alignment splitting */
  uint64_t payload_bytes;   /* bytes written per execution, bf16 images and duplicates included */
  uint64_t read_bytes;      /* bytes read per execution */
  uint64_t vector_bytes;    /* bytes written through 16-byte units (second destinations excluded) */
  uint64_t scalar_bytes;    /* bytes written element by element (second destinations excluded) */
  uint64_t n_chunks;        /* work chunks per execution */
  uint32_t n_src_bufs;
  uint32_t n_dst_bufs;
} emrs_plan_stats;

/* Description of the last failure on this thread ("" if none). */
const char *emrs_last_error(void);

/* EMRS_ABI_VERSION of the loaded library. */
int emrs_abi_version(void);

/* Number of visible HIP devices (0 when none); never fails. */
int emrs_device_count(void);

/*
 * Validate segments and build a plan.  Host-only: no device work is done
 * here (the table is uploaded on first execution).
 *   src_buf_bytes[i]: capacity in bytes of source buffer i (bounds check)
 *   dst_buf_bytes[i]: capacity in bytes of destination buffer i
 * Errors: INVALID_ARGUMENT (bad elem_bytes, rows == 0, dst_stride or
 * aux_stride < len, unknown buffer id, unknown flags, a cast on a non-fp32
 * segment), OUT_OF_BOUNDS (a row leaves its buffer), TOO_MANY_BUFFERS,
 * OVERLAP (with EMRS_PLAN_CHECK_DISJOINT; aux writes included).
 */
int emrs_plan_create(const emrs_segment *segs, uint64_t n_segs,
                     const uint64_t *src_buf_bytes, uint32_t n_src_bufs,
                     const uint64_t *dst_buf_bytes, uint32_t n_dst_bufs,
                     uint32_t flags, emrs_plan **out_plan);

int emrs_plan_stats_get(const emrs_plan *plan, emrs_plan_stats *out);

/*
 * Enqueue the plan on `stream`.  src_bases / dst_bases hold n_src_bufs /
 * n_dst_bufs device pointers.  Every buffer that a segment references must
 * be 16-byte aligned (EMRS_ERR_MISALIGNED) and must not overlap a referenced
 * buffer of the other side or another referenced destination buffer
 * (EMRS_ERR_ALIAS): the copy is out of place.  Unreferenced buffers are not
 * checked and may be NULL.  The first call on a device uploads the plan's
 * tables (segment table, chunk table and, beyond 128 buffers a side, its
 * pointer table for these bases) synchronously; later calls with the same bases enqueue the copy
 * kernel, preceded by the table pre-read of emrs_tuning.warm_tables, and
 * nothing else, so they may be captured into a HIP graph.  Calls with
 * other bases than the first beyond 128 buffers allocate a stream-ordered
 * pointer table.  Neither the first call nor such a call may be captured:
 * while `stream` is capturing they return EMRS_ERR_CAPTURE and enqueue
 * nothing.  Replaces one call of TransferManager.transfer_optimizer_tensors
 * (transfer.py:291-341) together with the bf16 rebuild of
 * TrainingState.update_model_weight (training_state.py:176-197).
 */
int emrs_plan_execute(emrs_plan *plan, void *const *src_bases,
                      void *const *dst_bases, void *stream);

/*
 * Do on the current device what the plan's first emrs_plan_execute there
 * would do before copying: upload the segment table and, when
 * emrs_tuning.chunk_index is on and emrs_tuning.persistent off (the
 * default), build the chunk table on the device.  Nothing is copied and no buffer is touched, so the first switch
 * then runs as fast as later ones.  Synchronous with `stream`; while it
 * captures a graph, EMRS_ERR_CAPTURE.  Replaces the reference's meta-device
 * pass, which runs a fake transfer to build its NCCL connections ahead of
 * the real switch (build_nccl_connection_context and its use in
 * ElasticMegatronManager.transfer_params, elastic_manager.py:115-117,
 * :282-304).
 */
int emrs_plan_prepare(emrs_plan *plan, void *stream);

/*
 * Free the plan.  Its device tables are freed in stream order after the
 * launches of emrs_plan_execute that use them (an event recorded after each
 * launch), so a plan may be destroyed while those launches are still queued;
 * the call neither blocks the host nor waits for other work on the device.
 * A plan whose launches were captured into a graph may be replayed at any
 * time, so for it the call first waits for the whole device; a graph that
 * holds its launches must not be replayed after the plan is destroyed.
 */
int emrs_plan_destroy(emrs_plan *plan);

/*
 * Verification of an executed plan: per group, how the destination differs
 * from what the plan would write there.
 *
 * The numbers are those of the reference's checkpoint check,
 * tools/ckpt/compare_ckpt.py:17-76 (max |a - b|, max |a - b| / (|b| + 1e-12),
 * RMS and relative RMS per tensor), plus an exact bit comparison.  The
 * reference first converts the source checkpoint on the CPU and then diffs
 * the two.  Here both states stay on the device: the plan supplies, for
 * every destination element, the source element (or zero) it must equal.
 * A cast segment's bf16 image is checked against bf16(source) as well.
 *
 * "expected" below is that value; "actual" is what the destination holds.
 * fp32 and bf16 elements (elem_bytes 4 and 2) are compared as numbers and
 * bit patterns; 1- and 8-byte elements as bit patterns only.
 */
typedef struct emrs_compare_stats {
  uint64_t elements;        /* elements compared */
  uint64_t mismatches;      /* elements whose bits differ from the expected value */
  uint64_t nonfinite;       /* mismatching fp32/bf16 elements with a NaN or infinite difference */
  uint64_t reserved;
  double sum_sq_diff;       /* sum of (actual - expected)^2 over finite differences */
  double sum_sq_expected;   /* sum of expected^2 over finite expected fp32/bf16 values; 0 for a group
                               without mismatches (its RMS and relative RMS are 0 either way) */
  float max_abs_diff;       /* max |actual - expected| over finite differences */
  float max_rel_diff;       /* max |actual - expected| / (|expected| + 1e-12) */
  uint64_t reserved2;
} emrs_compare_stats;

/*
 * Compare the destination buffers with what `plan` writes from the source
 * buffers, and accumulate the differences per group.  Two passes: the first
 * only finds the groups in which any bit differs, at the rate of a plain read;
 * only if there are such groups does a second pass compute every figure for
 * them.  A correct switch therefore costs one read of the source and the
 * destination.
 *   groups[i]:     group of input segment i's elements (NULL: all group 0)
 *   aux_groups[i]: group of input segment i's bf16 image (NULL: groups[i])
 *   stats:         n_groups host records, filled when the call returns
 * Base pointers follow emrs_plan_execute's rules, except that buffers may
 * overlap: a comparison only reads (a state that took over part of its
 * source's memory compares equal there).  The call runs on `stream`
 * and waits for it.  It allocates and frees a small device buffer (the
 * group tables and accumulators), so it is not for capture into a graph:
 * while `stream` is capturing it returns EMRS_ERR_CAPTURE.
 * Errors: INVALID_ARGUMENT (n_groups == 0, a group id >= n_groups), the
 * base-pointer errors of emrs_plan_execute but ALIAS, CAPTURE, NO_DEVICE, HIP.
 */
int emrs_plan_compare(emrs_plan *plan, void *const *src_bases, void *const *dst_bases,
                      const uint32_t *groups, const uint32_t *aux_groups, uint32_t n_groups,
                      emrs_compare_stats *stats, void *stream);

/*
 * emrs_plan_compare without any allocation.  No counterpart in the
 * reference: this entry point is for callers that cannot allocate device
 * memory (tight verification loops of an elastic controller, harnesses that
 * forbid hipMalloc).  Same arguments, checks and results as
 * emrs_plan_compare, but it calls no hipMalloc, hipFree or allocating
 * library routine: its accumulators, group ids, the plan's segment table and
 * (beyond 128 buffers a side) its pointer table are staged in a static device
 * array of EMRS_STATIC_SCRATCH_BYTES that every device holds until the
 * process ends.  A comparison that needs more (about 50,000 device segments
 * with few groups) returns EMRS_ERR_TOO_LARGE and does nothing.  The array is
 * shared by every call on a device and keeps the last call's contents; the
 * accumulators are cleared at the start of each call.  The library serialises
 * the calls of one process on one device, and each call waits for `stream`
 * before it returns, so calls never overlap in their use of the array.  Not
 * for capture into a graph (EMRS_ERR_CAPTURE).
 */
#define EMRS_STATIC_SCRATCH_BYTES (4u << 20)
int emrs_plan_compare_static(emrs_plan *plan, void *const *src_bases, void *const *dst_bases,
                             const uint32_t *groups, const uint32_t *aux_groups, uint32_t n_groups,
                             emrs_compare_stats *stats, void *stream);

/*
 * Launch-shape knobs of emrs_plan_execute, process-wide.  Results never
 * depend on them; only speed does.  By default every chunk of 256 units is
 * split into four pieces of 64 units (1 KB), one 64-lane workgroup each,
 * which finds its segment in the plan's chunk table; persistent = 1 selects
 * a persistent grid, which blocks_per_cu, run and xcd_remap shape.
 */
typedef struct emrs_tuning {
  uint32_t blocks_per_cu; /* workgroups per CU in the persistent grid (0..64);
                             0 (default): as many as can be resident at once */
  uint32_t nontemporal;   /* 1: streaming (non-temporal) loads and stores (default 1) */
  uint32_t xcd_remap;     /* 0, 1 (default) or 2.  Nonzero: each XCD works through one contiguous
                             eighth of the chunks (workgroup b runs on XCD b % 8); the persistent
                             grid does so for 1 and 2, one workgroup per piece for 2 and, with 1,
                             for plans of at least 2^19 chunks.  0: workgroup b takes piece b (one
                             workgroup per piece) or the b-th run (persistent) */
  uint32_t run;           /* persistent grid, 0: each workgroup copies one contiguous run of
                             chunks; N in [1, 2^20]: chunks are dealt out round-robin in runs of
                             8N, capped at a quarter of a workgroup's share (default 4) */
  uint32_t persistent;    /* 0 (default): one workgroup per piece of a chunk; 1: persistent grid */
  uint32_t lanes;         /* one workgroup per piece of a chunk: lanes per workgroup, 64, 128 or 256
                             (0: the default, 64) */
  uint32_t units;         /* 16-byte units per lane, 1 (default), 2 or 4, with lanes * units
                             dividing 256: a chunk of 256 units is split into 256 / (lanes * units)
                             pieces, one workgroup each (0: 256 / lanes, one workgroup per chunk) */
  uint32_t buffer_ops;    /* one workgroup per piece, 1: 16-byte units are moved with buffer
                             instructions (32-bit offsets from a per-piece base); 0: with 64-bit
                             global addresses */
  uint32_t chunk_index;   /* one workgroup per piece, 1 (default): each workgroup reads its
                             segment from the plan's chunk table (4 * emrs_plan_stats.n_chunks
                             bytes of device memory, made on the plan's first such call on a
                             device and freed with the plan; when that allocation runs out of
                             memory, the launch searches instead); 0: a binary search bounded by
                             a hint in the kernel arguments */
  uint32_t warm_tables;   /* with the chunk table, 1 (default): a short kernel reads the chunk table
                             and the segment descriptors just before each copy, so that the copy's
                             first load in every workgroup hits the memory-side cache even when the
                             launch follows unrelated work; 0: the copy alone */
} emrs_tuning;

int emrs_get_tuning(emrs_tuning *out);
int emrs_set_tuning(const emrs_tuning *t);

/*
 * Synthetic workload support (not on the reshard path).
 *
 * A piece is a run of one parameter's elements stored contiguously in a
 * buffer.  Element i of the piece is element (local_start + i) of the
 * parameter's TP-local tensor, laid out row-major with local_cols columns;
 * local (r, c) maps to the full tensor at
 *   row = (r < band_rows || band_rows == 0) ? r + row_off : r - band_rows + row_off2
 *   col = c + col_off
 * and full flat index row * full_cols + col.  band_rows splits the local rows
 * into two bands (fused SwiGLU [W; V]); 0 means one band.
 *
 * kind selects the value stream and storage type:
 *   0 param      bf16, ~N(0, 0.02)
 *   1 main       fp32, exact upcast of the kind-0 value
 *   2 exp_avg    fp32, ~N(0, 1e-3)
 *   3 exp_avg_sq fp32, |N(0, 1e-6)|
 * Every value is a pure function of (seed, param_id, kind, full flat index).
 */
typedef struct emrs_piece {
  uint32_t buf;
  uint32_t param_id;
  uint32_t kind;
  uint32_t reserved;
  uint64_t buf_off;     /* elements of the piece's storage type */
  uint64_t len;
  uint64_t local_start;
  uint64_t local_cols;
  uint64_t full_cols;
  uint64_t band_rows;
  uint64_t row_off;
  uint64_t row_off2;
  uint64_t col_off;
} emrs_piece;

/* Write the synthetic values of every piece into its buffer. */
/* emrs_synth_fill / emrs_synth_verify take at most 128 buffers. */
int emrs_synth_fill(const emrs_piece *pieces, uint64_t n_pieces,
                    void *const *bases, const uint64_t *buf_bytes,
                    uint32_t n_bufs, uint64_t seed, void *stream);

/*
 * Compare every piece with its synthetic values.  Synchronous: waits for
 * `stream`.  *mismatches receives the number of differing elements and
 * *first_bad the smallest (piece index << 40 | element index) that differs
 * (UINT64_MAX when none).
 */
int emrs_synth_verify(const emrs_piece *pieces, uint64_t n_pieces,
                      void *const *bases, const uint64_t *buf_bytes,
                      uint32_t n_bufs, uint64_t seed, void *stream,
                      uint64_t *mismatches, uint64_t *first_bad);

/*
 * XOR of every 32-bit word of the device buffer [p, p + bytes) into the
 * device word *out (zeroed first), enqueued on `stream`.  p and bytes must be
 * multiples of 16.  The buffer is read with 16-byte non-temporal loads in
 * the fastest read schedule found on MI355X, so the call also measures the
 * device's read-only HBM bandwidth.  No counterpart in the reference.
 */
int emrs_xor_checksum(const void *p, uint64_t bytes, uint32_t *out, void *stream);

/*
 * Inter-process hand-off.
 *
 * The reference passes a process's optimizer state to its successor with a
 * CUDA-IPC handle per tensor storage: _make_cuda_tensor_info packs each
 * storage's handle, size and offset (elastic_megatron/transfer/ipc_manager.py:23-51,
 * sent by send_training_state, :54-132) and receive_training_state rebuilds
 * the tensors from them (:135-155, rebuild_cuda_tensor).  Here the exporting
 * process holds its state in allocations of less than 2 GiB each, exports
 * each allocation once, and the importing process opens them and runs the
 * reshard straight from the mapped memory.
 *
 * An emrs_ipc_buffer is plain bytes: it can be written to a file, a pipe or
 * a socket and read back in another process on the same machine.
 */
#define EMRS_IPC_HANDLE_BYTES 64
#define EMRS_IPC_MAX_ALLOCATION_BYTES (2ull << 30) /* exclusive: allocations must be smaller */

typedef struct emrs_ipc_buffer {
  uint8_t handle[EMRS_IPC_HANDLE_BYTES]; /* hipIpcMemHandle_t of the allocation holding the buffer */
  uint64_t offset;           /* bytes from the allocation's base to the buffer (multiple of 16) */
  uint64_t bytes;            /* bytes of the buffer */
  uint64_t allocation_bytes; /* bytes of the whole allocation, < EMRS_IPC_MAX_ALLOCATION_BYTES */
  int32_t device;            /* device ordinal in the exporting process */
  uint32_t reserved;         /* must be 0 */
} emrs_ipc_buffer;

/*
 * Describe the device buffer [ptr, ptr + bytes) for another process: the
 * handle of the allocation that holds it and the buffer's place in it
 * (ipc_manager.py:23-51; the same fields as storage._share_cuda_'s handle,
 * size and offset).  The memory stays owned by the caller, who must keep it
 * allocated until every importer has closed it.
 * Errors: INVALID_ARGUMENT (NULL, empty, not device memory), MISALIGNED (ptr
 * not 16-byte aligned), TOO_LARGE (the allocation is 2 GiB or larger: it is
 * refused, not split), OUT_OF_BOUNDS, HIP.
 */
int emrs_ipc_export(const void *ptr, uint64_t bytes, emrs_ipc_buffer *out);

/*
 * Map an exported buffer into this process on the current device and return
 * its address in *ptr (ipc_manager.py:135-155).  Opening several buffers of
 * one allocation, or one buffer several times, maps the allocation once and
 * counts references.  The mapped memory is read and written like any device
 * buffer; pass it to emrs_plan_execute as a source base.  Must be called from
 * another process than the exporter's.
 * Errors: INVALID_ARGUMENT, TOO_LARGE (allocation_bytes of 2 GiB or more, or
 * 0: refused before the driver sees the handle), OUT_OF_BOUNDS, MISALIGNED,
 * HIP (the handle could not be opened).
 */
int emrs_ipc_open(const emrs_ipc_buffer *buf, void **ptr);

/*
 * Drop one reference that emrs_ipc_open returned; the allocation is unmapped
 * when its last reference goes.  The caller must first wait for the work
 * that uses the mapping.
 * Errors: INVALID_ARGUMENT (not a pointer emrs_ipc_open returned, or already
 * closed as many times as it was opened), HIP.
 */
int emrs_ipc_close(void *ptr);

/* Number of allocations this process holds open through emrs_ipc_open. */
int emrs_ipc_open_count(void);

#ifdef __cplusplus
}
#endif

#endif /* EMRS_H */
