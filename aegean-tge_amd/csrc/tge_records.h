// Plan records of the gfx950 paged-KV path: built on the host once per step
// (host/plan.cpp), uploaded once and read by every layer's kernels. Plain
// structs, shared by the host-only planner and the HIP translation units.
#pragma once

#include <stdint.h>

namespace tge {

constexpr int kPageTokens = 16;   // block_table.hpp:19 kBlockTokens
constexpr int kWaves = 4;         // waves per block-prefill workgroup
constexpr int kMaxRows = 64;      // query rows (n_new * group) per decode unit
constexpr int kPrefillRows = 128; // rows of one block-prefill work item (4 waves x 32)

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
};

static_assert(sizeof(WorkRec) == 12 * sizeof(int), "WorkRec is read as 12 ints");

// One row set whose context was split over several units.
struct ReduceRec {
  int session;
  int row_begin;
  int rows;
  int rows_per_query;
  int head_base;
  int first_part;
  int n_parts;
  int pad;
};

struct RowRec {  // one new token: destination page and slot, logical position
  int page;
  int slot;
  int pos;
};

}  // namespace tge
