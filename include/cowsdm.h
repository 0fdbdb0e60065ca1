/*
 * cowsdm.h -- C ABI of libcowsdm.so, the MI355X (gfx950) copy-on-write
 * Sparse Delta Memory (SDM) decode step and its state lifecycle.
 *
 * Every entry point takes device pointers, 64-bit sizes and a hipStream_t
 * (passed as void*), enqueues its kernels on that stream and returns 0 on
 * success.  A nonzero return is either a hipError_t or one of the negative
 * COWSDM_E* codes below; cowsdm_last_error_string() then describes it.
 * Nothing here allocates or frees device memory: callers own every buffer,
 * including the scratch and workspace arguments, whose sizes are given by
 * the *_words / *_bytes helpers.  Entry points never synchronise the stream.
 *
 * Layout of one SDM layer's packed state (the same tensors the reference's
 * PackedSDMCopyOnWriteState holds, copy_on_write_sdm/allocator.py:476-504):
 *   shared_initial_memory  float  [T, N, D]  model-shared M0, read only
 *   template_indices       int64  [B]        bank -> template row of M0
 *   values                 float  [C, D]     physical slab shared by banks
 *   logical_to_physical    int32  [B, N]     -1 = still shared with M0
 *   free_rows              int32  [C]        free stack, top = free_count-1
 *   free_count             int32  scalar
 *   overflow_flag          int32  scalar
 *   scratch                int64  [cowsdm_step_scratch_words(B)]  zeroed
 *                          once at creation; the step kernels keep it valid
 *
 * Index tensors (write/read routes) are int32 or int64, row-major [B, K].
 * Weights, values and gates are float32.  A bank is one (request, memory
 * head) pair.
 */
#ifndef COWSDM_H
#define COWSDM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define COWSDM_ABI_VERSION 12

/* Index dtype codes. */
#define COWSDM_INDEX_INT32 0
#define COWSDM_INDEX_INT64 1

/* Negative return codes (hipError_t values are positive). */
#define COWSDM_EARG (-1)      /* invalid argument (null pointer, bad size) */
#define COWSDM_ELIMIT (-2)    /* shape outside what the kernels support   */

/* Bits of the device error word (scratch word COWSDM_SCRATCH_ERRORS) and
 * of the precheck result word. */
#define COWSDM_ERR_WRITE_INDEX 0x1   /* write index outside [0, N)        */
#define COWSDM_ERR_READ_INDEX 0x2    /* read index outside [0, N)         */
#define COWSDM_ERR_DUP_WRITE 0x4     /* one step writes one slot twice    */
#define COWSDM_ERR_EXHAUSTED 0x8     /* free stack cannot cover the step  */
#define COWSDM_ERR_TEMPLATE 0x10     /* template index outside [0, T)     */
#define COWSDM_ERR_CORRUPT 0x20      /* map/free entry outside [0, C)     */
#define COWSDM_ERR_LOOKBACK 0x40     /* bank-order scan did not complete  */
#define COWSDM_ERR_TRACE_RANGE 0x80  /* trace step past steps_recorded    */

/* Word offsets inside the per-layer step scratch (int64 words). */
/* EPOCH retires the previous launch's scan slots (the layer's last wave
 * advances it); TICKET counts the waves of one-step launches that built
 * the layer's first-touch table themselves (every such launch adds the
 * bank count; a zeroed word starts it); ERRORS is the sticky COWSDM_ERR_*
 * word; SLOTS[b] is bank b's scan slot.  Words 2 and 4-7 are reserved. */
#define COWSDM_SCRATCH_EPOCH 0
#define COWSDM_SCRATCH_TICKET 1
#define COWSDM_SCRATCH_ERRORS 3
#define COWSDM_SCRATCH_SLOTS 8

/* Shape shared by every layer of one step launch. */
typedef struct cowsdm_shape {
  int64_t banks;        /* B: live banks                          */
  int64_t slots;        /* N: logical rows per bank               */
  int64_t width;        /* D: row width (floats)                  */
  int64_t writes;       /* W: write routes per bank, 1..64        */
  int64_t reads;        /* R: read routes per bank, 1..256        */
  int64_t templates;    /* T: rows of shared_initial_memory       */
  int32_t index_dtype;  /* COWSDM_INDEX_INT32 / COWSDM_INDEX_INT64 */
  int32_t reserved;
} cowsdm_shape_t;

/* One layer's tensors for a packed (or dense) step.  For the dense step,
 * `values` is the dense table [B, N, D] and the allocator fields
 * (logical_to_physical, free_rows, free_count, overflow_flag, scratch,
 * shared_initial_memory, template_indices, first/repeated/allocated) are
 * ignored and may be null. */
typedef struct cowsdm_layer {
  const float* shared_initial_memory;
  const int64_t* template_indices;
  float* values;
  int32_t* logical_to_physical;
  const int32_t* free_rows;
  int32_t* free_count;
  int32_t* overflow_flag;
  int64_t* scratch;
  int64_t capacity_rows;
  const void* write_indices;
  const float* write_weights;
  const float* step_values;
  const float* input_gate;
  const float* erase_gate;      /* may equal input_gate */
  const float* forget_log_gate;
  const void* read_indices;
  const float* read_weights;
  float* output;                /* [B, D] */
  int64_t* first_touches_out;   /* [B] or null */
  int64_t* repeated_writes_out; /* [B] or null */
  int32_t* allocated_rows_out;  /* scalar or null */
  /* Paged slot map (map_page_shift > 0; 0 keeps the direct map
   * logical_to_physical).  With P = 1 << map_page_shift slots per page,
   * bank b's slot x is mapped at
   *   map_pages[(map_directory[b * (N / P) + x / P] << map_page_shift) + x % P]
   * and a directory entry of -1 means no slot of that page is mapped.  Pages
   * in use are map_pages rows 0 .. *map_page_count - 1; a step takes new ones
   * from *map_page_count up (never more than map_page_capacity), at most one
   * per write route.  logical_to_physical is ignored (may be null).  Paged
   * layers run the one-step kernel only: W <= 4, R <= 16, D <= 256, B <= 256
   * (COWSDM_ELIMIT otherwise), and no persistent launches. */
  int32_t* map_directory;       /* [B, N / P] */
  int32_t* map_pages;           /* [map_page_capacity, P] */
  int32_t* map_page_count;      /* scalar */
  int64_t map_page_capacity;
  int32_t map_page_shift;
  int32_t map_reserved;
} cowsdm_layer_t;

/* Consecutive steps over device-resident inputs of many decode steps;
 * per-step inputs (and the output) sit at base + step * stride_bytes[k],
 * k in the order write_indices, write_weights, step_values, input_gate,
 * erase_gate, forget_log_gate, read_indices, read_weights, output, and the
 * inputs hold steps_recorded steps.
 *
 * Host offsets (step_index null): the call runs steps first_step ..
 * first_step + steps - 1 of every layer.
 *
 * Device counters (step_index set, nlayers int64 counters): layer l runs up
 * to `steps` steps from step_index[l], never past steps_recorded, and the
 * kernels advance step_index[l] by the steps it ran, so the call can be
 * captured once in a hipGraph and replayed.  A caller that knows where the
 * counters stand (every layer's the same) may say so: first_known nonzero
 * and the value in first_step.  Persistent launches then take their first
 * step from there rather than waiting for the counter's load before their
 * first input loads, and still compare it with the counter (a mismatch sets
 * COWSDM_TRACE_FAULT); a call of several launches does so for its first.  ticket points at 1 + nlayers
 * int64 words that are zero before the first launch and stay zero between
 * launches.  A layer with no step left runs nothing and sets
 * COWSDM_TRACE_ENDED in status[l] (status null, packed state:
 * COWSDM_ERR_TRACE_RANGE instead).
 *
 * Persistent launches: with persistent != 0 one launch runs up to
 * scan_steps (at most 512) steps when the shape allows it (W <= 4, R <= 16,
 * D <= 256, banks <= 256 for packed state, and every workgroup of one layer
 * resident; layers whose workgroups do not all fit at once run as groups of
 * layers, one launch after another), else one launch per step.
 *
 * Packed persistent launches plan each launch before running its steps,
 * inside the decode kernel: every bank's control wave counts its
 * (step, bank) first touches (a separate count kernel first when the slot
 * map does not fit in LDS) and scans a share of the steps across banks, and
 * one wave per layer replays the decode loop's capacity proof
 * (prepare_step_capacity(need) before every step, allocator.py:745-773,
 * inference.py:551-552), grows the slab within its buffer as grow_capacity
 * would (allocator.py:691-743), and lists the rows every first touch pops in
 * the order of single-step launches (step-major, bank-major within a step,
 * allocator.py:1471-1481), writing the free stack and free_count the launch
 * leaves.  The steps then take their rows from that list.  Readings, maps,
 * slab rows, free stacks and growth counters equal those of the loop of
 * single steps.  The proof state lives on the device in `control`
 * (COWSDM_CTRL_WORDS words per layer, word k of layer l at
 * control[k * control_stride + l]); the caller sets it before the launches
 * and reads it back after them.  `scan` holds nlayers blocks of scan_words
 * int64 words (>= cowsdm_trace_scan_words(banks, writes, scan_steps)) for
 * the plan. */
typedef struct cowsdm_trace {
  int64_t* step_index;
  int64_t* ticket;
  int64_t first_step;
  int64_t stride_bytes[9];
  int64_t* scan;
  int64_t scan_words;
  int32_t persistent;
  int32_t scan_steps;       /* steps per launch the scan blocks hold */
  int64_t steps_recorded;
  int32_t* status;          /* per-layer COWSDM_TRACE_* bits, or null */
  int64_t* control;         /* packed persistent launches, see above */
  int64_t control_stride;
  int64_t* report;          /* host-mapped report (COWSDM_REPORT_WORDS per layer), or null */
  int32_t first_known;      /* nonzero: every step_index[l] holds first_step (see above) */
  int32_t reserved;
} cowsdm_trace_t;

/* Control words of one layer of a packed decode trace (int64, word k of
 * layer l at control[k * control_stride + l]).  The caller sets them from
 * its state; a launch's plan reads and updates them.
 *   PROVEN    rows proven but not yet charged (the reference's
 *             proven_maximum_additional_allocations)
 *   CAPACITY  slab capacity C in rows (grows within ROOM)
 *   ROOM      rows of the slab's buffers (values and free_rows)
 *   QUANTUM   growth quantum in rows (0: no growth)
 *   NEED      rows proven before every step (banks * W), 0: no proof
 *   EVENTS, ADDED, COPIED  growth counters, added to by each launch
 *   FREE      free_count after the last launch
 *   STEPS     steps the last launch ran (its plan stops a layer before a
 *             growth past ROOM and sets COWSDM_TRACE_REFUSED)
 *   FIT       first touches of the last launch that got rows */
#define COWSDM_CTRL_PROVEN 0
#define COWSDM_CTRL_CAPACITY 1
#define COWSDM_CTRL_ROOM 2
#define COWSDM_CTRL_QUANTUM 3
#define COWSDM_CTRL_NEED 4
#define COWSDM_CTRL_EVENTS 5
#define COWSDM_CTRL_ADDED 6
#define COWSDM_CTRL_COPIED 7
#define COWSDM_CTRL_FREE 8
#define COWSDM_CTRL_STEPS 9
#define COWSDM_CTRL_FIT 10
#define COWSDM_CTRL_WORDS 12

/* The report a trace launch writes when trace->report is set: word k of
 * layer l at report[l * COWSDM_REPORT_WORDS + k], written by the layer's
 * last wave once every wave of the layer is done with the launch, into
 * host memory the device can write (cowsdm_host_report_alloc):
 *   0      the layer's step counter after the launch
 *   1      its status bits (COWSDM_TRACE_*)
 *   2 + k  control word k (packed persistent launches; 0 otherwise)
 * A host that waits for the launch's stream reads the layer's state there
 * without a device-to-host copy. */
#define COWSDM_REPORT_WORDS (2 + COWSDM_CTRL_WORDS)

/* Bits of a decode trace's per-layer status word (sticky: the kernels only
 * set them). */
#define COWSDM_TRACE_REFUSED 0x1  /* stopped before a growth past ROOM     */
#define COWSDM_TRACE_ENDED 0x2    /* no recorded step left                 */
#define COWSDM_TRACE_FAULT 0x4    /* stopped by a timed-out wait or corrupt
                                     state (see the scratch error word)    */

/* ---------------------------------------------------------------- info */

int32_t cowsdm_abi_version(void);
const char* cowsdm_last_error_string(void);
/* int64 words of step scratch one layer with `banks` banks needs. */
int64_t cowsdm_step_scratch_words(int64_t banks);
/* int64 words per layer of a packed decode trace's scan blocks for launches
 * of up to `steps` steps (cowsdm_trace_t.scan). */
int64_t cowsdm_trace_scan_words(int64_t banks, int64_t writes, int32_t steps);
/* 1 when trace launches of these layers run persistent (shape, pointer
 * alignment and strides allow it; see cowsdm_trace_t), else 0: packed
 * launches then need control null and run one launch per step.  No
 * counterpart in the reference. */
int32_t cowsdm_trace_persistent(const cowsdm_layer_t* layers, int32_t nlayers,
                                const struct cowsdm_shape* shape,
                                const struct cowsdm_trace* trace, int32_t dense);

/* Host memory the device can write, for trace reports: `words` int64
 * words, zeroed; *host is the host's address of it, *device the device's.
 * Free with cowsdm_host_report_free(host) once no launch writes it.  No
 * counterpart in the reference. */
int32_t cowsdm_host_report_alloc(int64_t words, int64_t** host, int64_t** device);
int32_t cowsdm_host_report_free(int64_t* host);

/* Kernel timing of persistent trace launches, for measurement (no
 * reference counterpart; one host thread): after cowsdm_trace_timing(1)
 * each persistent trace launch (up to 1,024) records HIP events on its
 * stream at the start of its first kernel (the count kernel of a packed
 * launch whose slot map stays in HBM, else the decode kernel), at the start
 * of its decode kernel and at the decode kernel's end (hipExtLaunchKernel).
 * cowsdm_trace_timing_read waits for them, returns the summed launch time
 * (first kernel's start to the decode kernel's end) and the summed
 * decode-kernel time in milliseconds and the number of launches, and
 * forgets them.  cowsdm_trace_timing(0) stops recording. */
int32_t cowsdm_trace_timing(int32_t enable);
int32_t cowsdm_trace_timing_read(double* launch_ms, double* kernel_ms, int32_t* launches);
/* Bytes of lifecycle workspace for a ranking over `entries` map entries
 * (release / trim / append / pack handoff / invariant checks). */
int64_t cowsdm_workspace_bytes(int64_t entries, int64_t capacity_rows);

/* ---------------------------------------------------------- decode step */

/* One fused copy-on-write step for one layer: resolve the W write routes
 * through the map, pop free rows for first touches in bank-major order,
 * copy M0 rows, apply the FP32 gated-delta update, then the weighted read
 * of R rows (which observes this step's writes).
 * Replaces _packed_sdm_cow_step_triton, copy_on_write_sdm/allocator.py:
 * 1179-1319 (kernel 74-229), with the torch semantics of 1466-1525. */
int32_t cowsdm_packed_step(const cowsdm_layer_t* layer,
                           const cowsdm_shape_t* shape, void* stream);

/* The same step for `nlayers` independent layers in one launch (all layers
 * share one shape).  No counterpart in the reference: a batched form of
 * cowsdm_packed_step for callers that already hold every layer's routes. */
int32_t cowsdm_packed_step_layers(const cowsdm_layer_t* layers,
                                  int32_t nlayers,
                                  const cowsdm_shape_t* shape, void* stream);

/* `steps` consecutive launches of cowsdm_packed_step_layers, each on the
 * decode step *trace->step_index names (see cowsdm_trace_t).  Fixed
 * arguments make the sequence capturable in one hipGraph.  No counterpart
 * in the reference: for callers holding routes of many steps, such as
 * synthetic-route benchmarks and teacher-forced decode. */
int32_t cowsdm_packed_step_trace(const cowsdm_layer_t* layers, int32_t nlayers,
                                 const cowsdm_shape_t* shape,
                                 const cowsdm_trace_t* trace, int32_t steps,
                                 void* stream);

/* cowsdm_packed_step_trace with the plan blocks in the library's own device
 * memory: trace->scan must be null (scan_words is ignored).  No counterpart
 * in the reference; for callers that cannot allocate device memory, such as
 * code under HIP graph capture and serving loops that forbid allocation.  It
 * allocates nothing: the plan blocks live in a static device array of
 * COWSDM_STATIC_SCAN_WORDS int64 words on each GPU (16 MiB, held until the
 * process ends), which limits a call to nlayers *
 * cowsdm_trace_scan_words(banks, W, scan_steps) words (COWSDM_ELIMIT
 * beyond).  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (other streams, other host threads) race.  A call whose
 * layout (banks, W, scan_steps, nlayers) differs from the last call's on the
 * GPU first zeroes the words it uses, with a kernel on `stream`.  A call
 * recorded into a hipGraph records that zeroing too (a fill kernel, no
 * memset node), and once one has been recorded on a GPU every later call
 * there zeroes its words first: a replay may have left another layout's
 * words in the array. */
#define COWSDM_STATIC_SCAN_WORDS (1ll << 21)
int32_t cowsdm_packed_step_trace_static(const cowsdm_layer_t* layers, int32_t nlayers,
                                        const cowsdm_shape_t* shape,
                                        const cowsdm_trace_t* trace, int32_t steps,
                                        void* stream);

/* The decode loop's launches for `steps` steps of every layer from their
 * device counters, `launch_steps` steps per launch (mode 0:
 * cowsdm_packed_step_trace, 1: cowsdm_packed_step_trace_static, 2:
 * cowsdm_dense_step_trace), then a wait: for a single launch until every
 * layer's report is in host memory (the kernel's waves may still be
 * exiting; later work on the stream waits for them), else for the stream.
 * trace->step_index and trace->report must be set: on return each layer's
 * report holds its step counter, status and control words after its last
 * launch.  No counterpart in the reference; its decode loop
 * (inference.py:538-566) calls one step at a time. */
int32_t cowsdm_trace_run(const cowsdm_layer_t* layers, int32_t nlayers,
                         const cowsdm_shape_t* shape, const cowsdm_trace_t* trace,
                         int64_t steps, int32_t launch_steps, int32_t mode, void* stream);

/* Dense-table control step on values = memory [B, N, D].
 * Replaces _dense_sdm_sparse_step_triton, allocator.py:1322-1378 (kernel
 * 367-460), with the torch semantics of 1612-1633. */
int32_t cowsdm_dense_step(const cowsdm_layer_t* layer,
                          const cowsdm_shape_t* shape, void* stream);
int32_t cowsdm_dense_step_layers(const cowsdm_layer_t* layers, int32_t nlayers,
                                 const cowsdm_shape_t* shape, void* stream);
/* Trace form of the dense control (see cowsdm_packed_step_trace). */
int32_t cowsdm_dense_step_trace(const cowsdm_layer_t* layers, int32_t nlayers,
                                const cowsdm_shape_t* shape,
                                const cowsdm_trace_t* trace, int32_t steps,
                                void* stream);

/* Route and capacity validation before a step; writes the COWSDM_ERR_*
 * bits it finds to *result (int64, device).  check_capacity counts the
 * step's first touches against free_count (packed state only).
 * Replaces _validate_indices / _validate_unique_writes (allocator.py:
 * 1107-1134) and the exhaustion assert of allocator.py:1279-1282, 1475. */
int32_t cowsdm_step_precheck(const cowsdm_layer_t* layer,
                             const cowsdm_shape_t* shape, int32_t dense,
                             int32_t check_unique, int32_t check_capacity,
                             int64_t* result, void* stream);

/* ------------------------------------------------------------ lifecycle */

/* Fresh state: map = -1, free_rows = 0..C-1, free_count = C, overflow = 0,
 * scratch = 0; template indices outside [0, T) set COWSDM_ERR_TEMPLATE in
 * *result.  Replaces PackedSDMCopyOnWriteState.allocate, allocator.py:
 * 506-585. */
int32_t cowsdm_init_state(int32_t* logical_to_physical, int64_t banks,
                          int64_t slots, int32_t* free_rows,
                          int64_t capacity_rows, int32_t* free_count,
                          int32_t* overflow_flag, int64_t* scratch,
                          int64_t scratch_words,
                          const int64_t* template_indices, int64_t templates,
                          int64_t* result, void* stream);

/* Slab growth: new_values[:old_C] = old_values; new_free_rows =
 * old free entries ++ (old_C .. new_C-1); free_count += new_C - old_C;
 * overflow = 0.  Replaces grow_capacity, allocator.py:691-743.  new_values
 * may be old_values (and new_free_rows old_free_rows): a slab allocated with
 * headroom grows in place, and no row moves. */
int32_t cowsdm_grow(const float* old_values, int64_t old_capacity,
                    float* new_values, int64_t new_capacity, int64_t width,
                    const int32_t* old_free_rows, int32_t* new_free_rows,
                    int32_t* free_count, int32_t* overflow_flag, void* stream);

/* Count entries >= 0 of map [banks, slots] rows bank_list[0..nsel) (rows
 * 0..nsel-1 when bank_list is null; listed rows outside [0, banks) count as
 * empty), row-major, or of active_mask [nsel, slots] when it is not null; writes the int64 total to *total and
 * keeps per-tile offsets in `workspace` for a following apply call on the
 * same map.  Replaces the `active.sum().item()` counts of allocator.py:628,
 * 791, 870 and the cumsum of 1057. */
int32_t cowsdm_count_active(const int32_t* logical_to_physical, int64_t banks,
                            int64_t slots, const int64_t* bank_list, int64_t nsel,
                            const uint8_t* active_mask, void* workspace,
                            int64_t* total, void* stream);

/* Pack a dense prefill terminal state: active (bank, slot) pairs of
 * active_mask [B, N] in row-major order get physical rows 0..A-1,
 * values[:A] = dense[bank, slot], free_rows[:C-A] = A..C-1,
 * free_count = C-A.  Needs cowsdm_count_active(mask) first.
 * Replaces the body of from_dense_overlay, allocator.py:664-685. */
int32_t cowsdm_pack_overlay(const float* dense_memory, const uint8_t* active_mask,
                            int64_t banks, int64_t slots, int64_t width,
                            int32_t* logical_to_physical, float* values,
                            int32_t* free_rows, int64_t capacity_rows,
                            int32_t* free_count, void* workspace, void* stream);

/* The handoff of several layers at once (from_dense_overlay of each,
 * allocator.py:587-689), in a few launches over all of them instead of
 * count, pack and invariant launches per layer.  One entry per layer:
 *   count part: dense_memory [B, N, D] float32, active_mask [B, N],
 *     workspace (cowsdm_workspace_bytes(B * N, max(B * N, capacity_rows))),
 *     total (int64: the layer's active entries A), template_indices [B]
 *     (templates rows of shared initial memory) and checks (9 int64 words:
 *     word 8 gets COWSDM_ERR_TEMPLATE or 0);
 *   pack part, after the caller has read the totals and allocated each
 *     layer's state: logical_to_physical [B, N], values [capacity_rows, D],
 *     free_rows [capacity_rows], free_count, overflow_flag, scratch
 *     (scratch_words int64).  The pack leaves the state of
 *     cowsdm_init_state + cowsdm_pack_overlay (free_rows[i] = A + i for
 *     i < C - A, i after), and checks words 0-7 get the counts of
 *     cowsdm_check_invariants.
 * No counterpart in the reference (its handoff is per layer, with host
 * reads of each layer's count and invariants). */
typedef struct cowsdm_handoff_layer {
  const float* dense_memory;
  const uint8_t* active_mask;
  int64_t banks, slots, width;
  void* workspace;
  int64_t* total;
  const int64_t* template_indices;
  int64_t templates;
  int64_t* checks;
  int32_t* logical_to_physical;
  float* values;
  int32_t* free_rows;
  int64_t capacity_rows;
  int32_t* free_count;
  int32_t* overflow_flag;
  int64_t* scratch;
  int64_t scratch_words;
} cowsdm_handoff_layer_t;

int32_t cowsdm_handoff_count(const cowsdm_handoff_layer_t* layers, int32_t nlayers,
                             void* stream);
int32_t cowsdm_handoff_pack(const cowsdm_handoff_layer_t* layers, int32_t nlayers,
                            void* stream);

/* Repack live rows into a smaller slab in row-major map order:
 * new_values[:A] = values[live rows], new_map = ranks, new_free_rows =
 * A..new_C-1, free_count = new_C - A, overflow = 0.  Needs
 * cowsdm_count_active(map) first.  Replaces trim_capacity,
 * allocator.py:775-839. */
int32_t cowsdm_trim_repack(const int32_t* logical_to_physical,
                           const float* values, int64_t capacity_rows,
                           int64_t banks, int64_t slots,
                           int64_t width, int32_t* new_logical_to_physical,
                           float* new_values, int32_t* new_free_rows,
                           int64_t new_capacity, int32_t* free_count,
                           int32_t* overflow_flag, void* workspace,
                           void* stream);

/* Admit another pool's banks: pop destination rows from the top of this
 * free stack in the other map's row-major live order, copy their values,
 * build new_map = [map ; admitted map] and new_templates = [templates ;
 * other templates], free_count -= A.  Needs cowsdm_count_active(other map)
 * first; the workspace holds cowsdm_workspace_bytes(other_banks * N,
 * other_capacity_rows).  Replaces append_banks_from, allocator.py:841-914. */
int32_t cowsdm_append_banks(const int32_t* logical_to_physical,
                            const int64_t* template_indices, int64_t banks,
                            float* values, int64_t capacity_rows,
                            const int32_t* free_rows, int32_t* free_count,
                            const int32_t* other_logical_to_physical,
                            const int64_t* other_template_indices,
                            const float* other_values, int64_t other_banks,
                            int64_t other_capacity_rows, int64_t slots,
                            int64_t width, int32_t* new_logical_to_physical,
                            int64_t* new_template_indices, void* workspace,
                            void* stream);

/* Validate bank indices for release / retain: bounds, duplicates, and (for
 * retain, when discarded_active != 0) whether any bank not listed still
 * owns rows.  Writes bits 1 (invalid or duplicated) and 2 (discarded bank
 * live) to *result.  Replaces the checks of allocator.py:1032-1051 and
 * 926-940. */
int32_t cowsdm_check_banks(const int32_t* logical_to_physical, int64_t banks,
                           int64_t slots, const int64_t* bank_list,
                           int64_t nsel, int32_t discarded_active,
                           void* workspace, int64_t* result, void* stream);

/* Release banks bank_list[0..nsel): push their live rows on the free stack
 * in (listed bank, slot) order, free_count += released, map rows = -1,
 * *released = count.  Needs cowsdm_count_active(map, bank_list) first.
 * Replaces release, allocator.py:1018-1067. */
int32_t cowsdm_release(int32_t* logical_to_physical, int64_t banks, int64_t slots,
                       const int64_t* bank_list, int64_t nsel,
                       int32_t* free_rows, int64_t capacity_rows,
                       int32_t* free_count, void* workspace, int64_t* released,
                       void* stream);

/* Keep banks bank_list[0..nsel) in that order: new_map[i] = map[list[i]],
 * new_templates[i] = templates[list[i]].  Values never move.
 * Replaces retain_banks, allocator.py:916-942. */
int32_t cowsdm_retain_banks(const int32_t* logical_to_physical,
                            const int64_t* template_indices, int64_t banks,
                            int64_t slots,
                            const int64_t* bank_list, int64_t nsel,
                            int32_t* new_logical_to_physical,
                            int64_t* new_template_indices, void* stream);

/* ---- paged slot maps (the compressed map the reference leaves for large
 * address spaces, README.md:123-130; allocator.py:485-489 reserves the
 * place: "a later compressed map can replace it without changing SDM").
 * A paged map holds the same entries as the direct map [B, N], in pages of
 * P = 1 << page_shift slots (P divides N); only pages with a mapped slot
 * exist (see cowsdm_layer_t).  Lifecycle operations run on the direct form:
 * cowsdm_paged_expand rebuilds it, cowsdm_paged_count + _compress pack it
 * back, pages numbered in row-major (bank, page) order. */

/* The pages holding a mapped slot: flags[b * (N / P) + g] = 1 when page g
 * of bank b holds one (uint8 [B * N / P]), and *total their count.  Leaves
 * the ranks cowsdm_paged_compress uses in `workspace`
 * (cowsdm_workspace_bytes(B * N / P, 0) bytes).  No counterpart in the
 * reference. */
int32_t cowsdm_paged_count(const int32_t* logical_to_physical, int64_t banks, int64_t slots,
                           int32_t page_shift, uint8_t* flags, void* workspace,
                           int64_t* total, void* stream);

/* After cowsdm_paged_count with the same arguments: directory[b, g] = the
 * page's rank among flagged pages (row-major), or -1; pages[rank] = the
 * map's P entries; *page_count = the flagged pages.  Size `pages` from the
 * count's total: pages ranked at or past page_capacity are not written.
 * No counterpart in the reference. */
int32_t cowsdm_paged_compress(const int32_t* logical_to_physical, int64_t banks,
                              int64_t slots, int32_t page_shift, const uint8_t* flags,
                              void* workspace, int32_t* directory, int32_t* pages,
                              int64_t page_capacity, int32_t* page_count, void* stream);

/* The direct map [B, N] of a paged one.  No counterpart in the reference. */
int32_t cowsdm_paged_expand(const int32_t* directory, const int32_t* pages,
                            int64_t page_capacity, int64_t banks, int64_t slots,
                            int32_t page_shift, int32_t* logical_to_physical, void* stream);

/* dense[b, n] = map[b, n] >= 0 ? values[map[b, n]] : M0[template[b], n].
 * Replaces materialize_dense, allocator.py:1003-1016. */
int32_t cowsdm_materialize_dense(const float* shared_initial_memory,
                                 int64_t templates,
                                 const int64_t* template_indices,
                                 const float* values,
                                 const int32_t* logical_to_physical,
                                 int64_t banks, int64_t slots, int64_t width,
                                 int64_t capacity_rows, float* dense,
                                 void* stream);

/* Partition check of live and free rows.  Writes 8 int64 words to stats:
 * [0] live rows, [1] free rows, [2] rows with two or more live owners,
 * [3] rows listed twice on the free stack, [4] rows neither live nor free
 * exactly once, [5] entries outside [0, C), [6] overflow flag,
 * [7] step error word.  Replaces validate_invariants, allocator.py:
 * 1069-1095. */
int32_t cowsdm_check_invariants(const int32_t* logical_to_physical,
                                int64_t banks, int64_t slots,
                                const int32_t* free_rows,
                                const int32_t* free_count,
                                const int32_t* overflow_flag,
                                const int64_t* scratch,
                                int64_t capacity_rows, void* workspace,
                                int64_t* stats, void* stream);

/* active_mask[b, idx[b, k]] = 1 for k < K (indices outside [0, N) are
 * ignored and reported as 0x2 in *result when result is not null).  The prefill handoff's union of
 * written rows, inference.py:332-347. */
int32_t cowsdm_mark_written(uint8_t* active_mask, int64_t banks, int64_t slots,
                            const void* indices, int64_t per_bank,
                            int32_t index_dtype, int64_t* result,
                            void* stream);

/* Product-key routes, sdm.py:96-159 (product_key_routes; called for the
 * write and read routes of a decode step at inference.py:479-488).
 * projected is [rows, 2*sqrt(slots)] float32: each row's two halves are
 * shortlisted to their top min(selected, sqrt(slots)) scores, the pair sums
 * ranked, and the best K = min(selected, min(selected, sqrt(slots))^2) pairs
 * written as slots first*sqrt(slots)+second, ascending, to indices[rows, K]
 * (int64) with the softmax of their scores in weights[rows, K].  Equal scores
 * are taken lowest position first; inputs must be finite.  Returns -1 for the
 * reference's argument errors (slots not a square, selected outside
 * [1, slots]) and -2 beyond the HIP path's limits (sqrt(slots) <= 1024,
 * min(selected, sqrt(slots)) <= 32, K <= 32). */
int32_t cowsdm_product_key_routes(const float* projected, int64_t rows,
                                  int64_t slots, int64_t selected,
                                  float* weights, int64_t* indices,
                                  void* stream);

/* ----------------------------------------------------- controller step */

/* Weights of one SDM layer's controller (float32, device; SparseDeltaMemory,
 * sdm.py:998-1052).  Projection weights are stored transposed, [in, out]:
 * proj_weight_t [width, rows] holds, in this order, the read keys
 * (heads x 2*sqrt(slots)), the write keys (the same), the values (width),
 * the forget gates (heads) and the input gates (heads) of read_projection,
 * write_projection, value_projection, forget_projection and
 * input_projection (rows = cowsdm_controller_rows(width, heads, slots)). */
typedef struct cowsdm_controller {
  int64_t width;            /* model width, heads * head_width       */
  int64_t heads;            /* memory heads                          */
  int64_t slots;            /* N, a perfect square                   */
  const float* norm_weight; /* input_norm (LayerNorm(width))         */
  const float* norm_bias;
  const float* proj_weight_t;   /* [width, rows]                     */
  const float* proj_bias;       /* [rows]                            */
  const float* a_log;           /* [heads]                           */
  const float* dt_bias;         /* [heads]                           */
  const float* gate_weight_t;   /* output_gate, [width, width]       */
  const float* gate_bias;
  const float* out_weight_t;    /* output_projection, [width, width] */
  const float* out_bias;
  const float* read_norm_weight;  /* readings_norm (LayerNorm(head_width)) */
  const float* read_norm_bias;
  float norm_eps;
  float read_norm_eps;
} cowsdm_controller_t;

/* Rows of the fused controller projection, or -1 for invalid sizes. */
int64_t cowsdm_controller_rows(int64_t width, int64_t heads, int64_t slots);

/* The position-parallel part of _prepare_faithful_sdm_step
 * (inference.py:459-519) for `batch` tokens [batch, width]: normalized
 * [batch, width] = input_norm(tokens); read and write keys
 * [batch * heads, 2*sqrt(slots)]; values [batch * heads, head_width];
 * input_gate = sigmoid(input_projection) and forget_log_gate =
 * -exp(A_log) * softplus(forget_projection + dt_bias), [batch * heads];
 * row b * heads + h for token b and head h.  Routes come from the keys
 * through cowsdm_product_key_routes.  width <= 1024. */
int32_t cowsdm_controller_prepare(const cowsdm_controller_t* controller, const float* tokens,
                                  int64_t batch, float* normalized, float* read_keys,
                                  float* write_keys, float* values, float* input_gate,
                                  float* forget_log_gate, void* stream);

/* _finish_faithful_sdm_step (inference.py:522-535): out [batch, width] =
 * output_projection(sigmoid(output_gate(normalized)) *
 * readings_norm(reading)), the reading [batch * heads, head_width]
 * normalised per head. */
int32_t cowsdm_controller_finish(const cowsdm_controller_t* controller,
                                 const float* normalized, const float* reading,
                                 int64_t batch, float* out, void* stream);

/* cowsdm_controller_prepare followed by the product-key routes of every
 * token's read and write keys (sdm.py:96-159, as
 * _prepare_faithful_sdm_step calls them, inference.py:479-488), in one
 * launch when sqrt(slots) <= 64: read_weights/read_indices
 * [batch * heads, min(reads, min(reads, sqrt N)^2)], the write routes
 * likewise; larger tables fall back to the three separate launches.  The
 * routes equal cowsdm_product_key_routes' bit for bit; reads and writes
 * take its `selected` checks.  No single counterpart in the reference: it
 * is the fusion of the calls above for a decode step's launch count. */
int32_t cowsdm_controller_prepare_routes(
    const cowsdm_controller_t* controller, const float* tokens, int64_t batch,
    float* normalized, float* read_keys, float* write_keys, float* values, float* input_gate,
    float* forget_log_gate, int64_t reads, int64_t writes, float* read_weights,
    int64_t* read_indices, float* write_weights, int64_t* write_indices, void* stream);

/* cowsdm_controller_finish that also writes out_sum = residual + out
 * [batch, width] (the residual add after the SDM mixer, tokens + mixed,
 * inference.py:660) when residual is non-null; out is written either
 * way. */
int32_t cowsdm_controller_finish_residual(const cowsdm_controller_t* controller,
                                          const float* normalized, const float* reading,
                                          int64_t batch, float* out, const float* residual,
                                          float* out_sum, void* stream);

/* One layer's cowsdm_controller_finish_residual (residual and out_sum
 * required) followed by the next layer's cowsdm_controller_prepare_routes
 * on out_sum: the layer stack's per-token walk (inference.py:655-661) for
 * a caller with nothing between the layers (the reference's stack puts an
 * MLP there, inference.py:661, and takes the two calls), in one launch
 * when the next layer's
 * sqrt(slots) <= 64 (its tokens' inputs stay on chip between the two), else
 * in the two launches.  The layers share their width.  Every output equals
 * the two calls' bit for bit.  No single counterpart in the reference. */
int32_t cowsdm_controller_finish_prepare_routes(
    const cowsdm_controller_t* controller, const float* normalized, const float* reading,
    int64_t batch, float* out, const float* residual, float* out_sum,
    const cowsdm_controller_t* next, float* next_normalized, float* read_keys,
    float* write_keys, float* values, float* input_gate, float* forget_log_gate,
    int64_t reads, int64_t writes, float* read_weights, int64_t* read_indices,
    float* write_weights, int64_t* write_indices, void* stream);

/* ------------------------------------------ dense recurrence (prefill) */

/* One SDM layer's token-serial recurrence over dense route vectors
 * (float32, device, contiguous).  Replaces _native_sdm_forward_kernel
 * (sdm.py:534-607) as _NativeSDMRecurrence.forward launches it
 * (sdm.py:779-861; gated_delta_recurrence, sdm.py:962-995).  Per batch row b
 * and token t: memory rows with a nonzero write route decay by
 * exp(forget_log_gate[b, t]); retrieved = sum_n write_routes * memory;
 * memory += write_routes * (input_gate * values - erase_gate * retrieved);
 * readings[b, t] = sum_n read_routes * memory. */
typedef struct cowsdm_recurrence {
  int64_t batch;                /* B                                   */
  int64_t time;                 /* T                                   */
  int64_t slots;                /* N <= 1024                           */
  int64_t width;                /* D                                   */
  const float* initial_memory;  /* [B, N, D]                           */
  const float* write_routes;    /* [B, T, N]                           */
  const float* values;          /* [B, T, D]                           */
  const float* input_gate;      /* [B, T]                              */
  const float* erase_gate;      /* [B, T]                              */
  const float* forget_log_gate; /* [B, T]                              */
  const float* read_routes;     /* [B, T, N]                           */
  float* readings;              /* [B, T, D]                           */
  float* states;                /* [B, T, N, D] per-token memory, or null */
  float* final_memory;          /* [B, N, D], or null                  */
} cowsdm_recurrence_t;

/* Runs the recurrence of cowsdm_recurrence_t; COWSDM_ELIMIT for N > 1024
 * (the reference's "at most 1,024 slots"). */
int32_t cowsdm_recurrence_forward(const cowsdm_recurrence_t* recurrence, void* stream);

/* Dense route vectors from sparse routes, sdm.py:162-172
 * (dense_sparse_routes): dense [rows, slots] = 0 except
 * dense[row, indices[row, k]] = weights[row, k] (the last k wins for a
 * repeated index).  An index outside [0, slots) sets bit 0x1 of *bad
 * (device int32, not cleared here; may be null). */
int32_t cowsdm_dense_routes(const float* weights, const void* indices, int32_t index_dtype,
                            int64_t rows, int64_t per_row, int64_t slots, float* dense,
                            int32_t* bad, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* COWSDM_H */
