// Host-side planning of one step of the gfx950 paged-KV path: validation of
// a batch description, the decode and block-prefill work lists, and the
// staged host->device upload of the plan. Plain C++ with no HIP types: the
// device side is reached through MemOps, so the planner also builds and runs
// on a CPU-only host (the sanitizer tests link it with a fake MemOps).
#pragma once

#include <cstddef>
#include <functional>
#include <vector>

#include "../csrc/tge_records.h"

namespace tge::plan {

// Device memory, pinned host memory, copies and ordering, as status-returning
// calls (TGE_OK or a tge_status). A stream or event is an opaque handle.
struct MemOps {
  virtual ~MemOps() = default;
  virtual int host_alloc(char** p, std::size_t bytes) = 0;
  virtual void host_free(char* p) = 0;
  virtual int dev_alloc(char** p, std::size_t bytes) = 0;
  virtual void dev_free(char* p) = 0;
  virtual int copy_to_device(char* dev, const char* host, std::size_t bytes, void* stream) = 0;
  // Record a marker after the work queued on `stream` (creating it when
  // *event is null); wait for a marker; wait for a stream.
  virtual int record(void** event, void* stream) = 0;
  virtual int wait_event(void* event) = 0;
  virtual int wait_stream(void* stream) = 0;
  virtual void event_free(void* event) = 0;
};

// A device buffer filled from pinned host staging. Both grow on demand and
// are reused across uploads. The recorded capacities always describe
// buffers that exist: a failed allocation leaves the buffer empty (capacity
// 0), so a later, smaller upload allocates again instead of writing through
// a freed pointer.
struct Staged {
  char* host = nullptr;
  std::size_t host_bytes = 0;
  char* dev = nullptr;
  std::size_t dev_bytes = 0;
  void* staged = nullptr;  // marker after the last copy out of `host`

  // Copy `bytes` (at least 256) written by `fill` into the host buffer to
  // the device buffer on `stream`. Waits for the previous copy out of the
  // host buffer first.
  int upload(MemOps& m, std::size_t bytes, void* stream, const std::function<void(char*)>& fill);
  void release(MemOps& m);
};

// A device array that grows on demand (split-K partials). Same capacity
// rule as Staged.
struct Scratch {
  char* dev = nullptr;
  std::size_t bytes = 0;
  // Make room for `need` bytes; waits for `stream` before freeing a smaller
  // buffer that queued work may still use.
  int reserve(MemOps& m, std::size_t need, void* stream);
  void release(MemOps& m);
};

// The sessions of one step (host copies of the plan records).
struct Step {
  std::vector<SessionRec> sessions;
  std::vector<int> tables;
  std::vector<RowRec> rows;
  int kv_heads = 0;
  int head_dim = 0;
  int block_dims = 0;  // width of the page blocks: 64, 128 or 256 (block_dims_for)
  int q_heads = 0;
  int group = 1;
  int pages = 0;     // pages of the pool
  int max_rows = 0;  // largest n_new * group
};

// Builds `step` from a batch description (the fields of tge_batch_desc),
// validating every rule first; on failure returns TGE_ERR_INVALID with a
// message and leaves `step` untouched.
int build_step(Step& step, int n_sessions, const int* ctx, const int* n_new,
               const int* table_offsets, const int* page_ids, int q_heads, int kv_heads,
               int head_dim, int pool_pages, const char** message);

// Work lists of one attention kind for the current step.
struct AttnLists {
  std::vector<WorkRec> work;
  std::vector<ReduceRec> reduce;
  std::vector<int> wg_first;  // [groups + 1] first item of each workgroup, or empty
  int groups = 0;             // workgroups of the launch
  int row_groups = 1;         // 16-row groups per unit
  int tile_rows = 0;          // prefill: rows of a tile (prefill_tile_rows, or 64)
  int parts = 0;              // split-K partial slots
  int max_splits = 0;
  // Decode launches that store the step's new rows (build_decode_appends):
  // the rows each wave stores, those of the pages it reads itself, as
  // records {page id, position, k/v row * kv_heads + KV head, work item};
  // wave w of workgroup g stores records [app_first[g*app_waves + w],
  // app_first[g*app_waves + w + 1]). kAppPad zero records follow the last.
  // app_waves 0: no lists (the launch cannot store the rows).
  std::vector<int> app_first;
  std::vector<int> app_recs;
  int app_waves = 0;
};


// Resident workgroups of the decode launch and the device's compute units;
// workgroup g is the (g / cus)-th to land on its compute unit.
struct Residency {
  int groups;
  int cus;
};

// Sessions a decode unit holds (n_new * group <= kMaxRows); `only`: 0 every
// session, 1 those, 2 the others.
bool decode_session(const Step& s, const SessionRec& r);
bool take_session(const Step& s, const SessionRec& r, int only);

// Decode schedule: every (session, KV head) is a segment of pages; the
// segments are laid end to end and cut into one share per resident
// workgroup (balanced by pages, per-piece cost and dispatch rank); a
// segment cut into several items is merged by the split reduction.
void build_decode(const Step& s, Residency res, AttnLists& out, int only);

// The new-row records of a decode plan whose launch of `waves` waves per
// workgroup stores the rows: page j (from page_begin) of work item `item`
// is read by wave (j + item) mod waves, which stores the new rows that page
// holds. No lists
// (app_waves 0) when `waves` is 0 or a wave would hold more than max_rows.
void build_decode_appends(const Step& s, AttnLists& pl, int waves, int max_rows);

// Block-prefill work: (session, KV head, query tile) x page splits sized so
// the launch covers `cus` compute units about twice; longest items first.
// `halves`: groups of four waves per workgroup (2: an item's pages are
// shared by two halves, so items may be twice as long). At 128 dims with
// two halves the tiles may be 64 rows (tile_rows) when 128-row tiles would
// leave compute units idle; `i8`: int8 pages (whose dequantisation makes a
// page read serve fewer rows at a higher cost, so unsplit 64-row tiles do
// not replace split 128-row ones).
void build_prefill(const Step& s, int cus, AttnLists& out, int only, int halves = 1,
                   bool i8 = false);

// A small decode step in one launch (paged_step_kernel): one workgroup per
// piece of a (session, KV head) segment; pieces of a split segment own
// consecutive partial slots and the segment's arrival counter.
struct StepLists {
  std::vector<StepRec> recs;
  std::vector<int> first_ids;  // [recs][kStepFirstIds]
  int row_groups = 1;
  int piece_pages = 0;  // pages of every piece but a segment's first
  int parts = 0;        // partial slots
  int segments = 0;     // arrival counters
  int max_pieces = 0;
};

// Builds the one-launch lists when every session's rows fit a decode unit
// (at most 48 rows at head_dim above 64) and the step holds at most
// kStepMaxBlocks page blocks; returns false (and leaves `out` empty)
// otherwise. Pieces are whole batches of the kernel's page loads
// (kStepWaves x step_batch_pages), at most kStepMaxParts per segment; the
// segment's last piece holds every page with a new position and stores the
// new rows.
constexpr int kStepMaxBlocks = 4096;
bool build_step_lists(const Step& s, bool i8, bool scale_f32, StepLists& out);

// The plan image of `lists` (work | reduce | wg_first, each 256-aligned):
// total bytes and the offsets of the reduce and wg_first parts.
// [ work | reduce | wg_first | app_first | app_recs ], each part 256-byte aligned.
std::size_t image_layout(const AttnLists& lists, std::size_t* off_reduce, std::size_t* off_first,
                         std::size_t* off_app = nullptr);
void write_image(const AttnLists& lists, std::size_t off_reduce, std::size_t off_first, char* dst,
                 std::size_t off_app = 0);

}  // namespace tge::plan
