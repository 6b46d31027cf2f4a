// Plan records of the gfx950 paged-KV path: built on the host once per step
// (host/plan.cpp), uploaded once and read by every layer's kernels. Plain
// structs, shared by the host-only planner and the HIP translation units.
#pragma once

#include <stdint.h>

namespace tge {

constexpr int kPageTokens = 16;   // block_table.hpp:19 kBlockTokens
constexpr int kWaves = 4;         // waves per block-prefill workgroup
constexpr int kMaxRows = 64;      // query rows (n_new * group) per decode unit
// Query rows of one decode unit at a block width: 64, or 48 in 256-dim
// blocks (three row groups: their Q^T table and two 16 KB ring slots per
// wave fill the CU's LDS).
constexpr int max_unit_rows(int block_dims) { return block_dims > 128 ? 48 : kMaxRows; }
constexpr int kPrefillRows = 128; // rows of one block-prefill work item (4 waves x 32)
// Rows of a block-prefill tile at a block width: 4 waves x 32 rows, or x 16
// rows in 256-dim blocks (a wave's accumulators for 32 rows would not fit).
constexpr int prefill_tile_rows(int block_dims) { return block_dims > 128 ? 64 : kPrefillRows; }

struct SessionRec {
  int ctx;        // positions cached before this step
  int n_new;      // new tokens (query rows per head) this step
  int q_row;      // first row of the session in q/k/v/out
  int table_off;  // first entry of the session's block table
};

// One attention workgroup: a session, a KV head, up to 16*NRG query rows and a
// range of logical pages. Row r is query row_begin + r / rows_per_query of
// head head_base + r % rows_per_query (decode: the GQA group of each new
// token; prefill: consecutive queries of one head).
struct WorkRec {
  int session;
  int kv_head;
  int page_begin;  // logical page range [page_begin, page_end)
  int page_end;
  int part;        // partial slot, or -1 when the unit writes the output
  int row_begin;
  int rows;
  int rows_per_query;
  int head_base;
  // copies of the session record, so a unit needs no second lookup
  int ctx;
  int q_row;
  int table_off;
  int red;  // reduction record of a split item (its partial's merge), or -1
  int pad[3];
};

static_assert(sizeof(WorkRec) == 16 * sizeof(int), "WorkRec is read as 16 ints");

// One row set whose context was split over several units.
struct ReduceRec {
  int session;
  int row_begin;
  int rows;
  int rows_per_query;
  int head_base;
  int first_part;
  int n_parts;
  int q_row;  // the session's first row in q/out (its SessionRec copy)
};

// One workgroup of a small decode step (append, attention and split merge
// in one launch): a piece of one (session, KV head) segment. The piece
// holding the segment's new positions stores the new rows of its KV head
// first; a segment cut into several pieces is merged by the last of its
// pieces to finish, found through the segment's arrival counter.
struct StepRec {
  int session;
  int kv_head;
  int page_begin;  // logical page range [page_begin, page_end)
  int page_end;
  int part;        // partial slot of this piece, or -1 (the segment is one piece)
  int seg;         // segment index: its arrival counter
  int seg_parts;   // pieces of the segment
  int seg_first;   // partial slot of the segment's first piece
  int append;      // 1: store the session's new rows of this KV head first
  int ctx;
  int n_new;
  int q_row;
  int table_off;
  int pad[3];
};

static_assert(sizeof(StepRec) == 16 * sizeof(int), "StepRec is read as 16 ints");

// The one-kernel decode step: waves per workgroup, and the pages one wave
// holds in registers at once (page images of 2*KW + 2*SW dwords per lane
// beside the unit's accumulators; KW dwords of K per lane = 16 tokens x
// head_dim elements / 64 lanes, SW dwords of scales). A piece of a context
// is a whole number of such batches. int8 pages take two per wave even
// where four fit: split contexts then have pieces half as long (the page
// math of a piece, not its loads, sets its length).
constexpr int kStepWaves = 8;
constexpr int kStepMaxParts = 64;  // pieces of one (session, KV head) context
// Page ids of a piece's first batch, stored beside its record so that the
// kernel loads them with the record instead of after it: [i][wave] is the
// i-th page of the wave's batch, page_begin + wave + i * kStepWaves, or the
// piece's last page past its end (batches hold at most 4 pages per wave).
constexpr int kStepFirstIds = 4 * kStepWaves;
constexpr int step_batch_pages(bool i8, bool scale_f32, int head_dim, int row_groups) {
  const int np = head_dim / 32;
  const int kw = i8 ? 2 * np : 4 * np;
  const int sw = i8 ? (scale_f32 ? 4 * np : 2 * np) : 0;
  return row_groups >= 3 || head_dim > 128 ? 1 : (2 * kw + 2 * sw <= 16 && !i8 ? 4 : 2);
}

// Steps the one-kernel step takes: rows per unit that fit its registers
// (`sparse`: the variant that applies a static sparse subset, whose extra
// row state spills with int8 pages and fp32 scales beyond 16 rows at 128
// dims and at 256 dims).
constexpr bool step_fits(bool i8, bool scale_f32, int head_dim, int rows, bool sparse = false) {
  if (rows > kMaxRows) return false;
  if (head_dim <= 64) return true;
  if (sparse && i8 && scale_f32) return head_dim <= 128 && rows <= 16;
  return rows <= (head_dim > 128 ? 16 : (i8 && scale_f32 ? 32 : 48));
}

// New-row records of a decode launch that stores the step's rows: ints per
// record ({page id, position, k/v row * kv_heads + KV head, work item}),
// and the zero records after the last list (a wave reads kAppPad records
// from its first).
constexpr int kAppRecInts = 4;
constexpr int kAppPad = 16;

struct RowRec {  // one new token: destination page and slot, logical position
  int page;
  int slot;
  int pos;
};

}  // namespace tge
