// Kernel parameter blocks and launchers shared by the API layer and the
// kernel translation units. Internal to libtge_kv.so.
#pragma once

#include <hip/hip_runtime.h>

#include "tge_common.h"

namespace tge {

// Head sizes: `dims` is the model's head_dim (the row stride of q, k, v,
// out and the biases); `head_dim` where it remains is the page blocks'
// width (block_dims_for), whose dims from `dims` on are stored as zeros.
struct AppendParams {
  const float* k;  // [n_rows][kv_heads*dims]
  const float* v;
  void* pool;      // layer base: the layer's page blocks
  BlockGeom geom;
  const RowRec* rows;  // device, n_rows
  int n_rows;
  int kv_heads;
  int head_dim;  // block width
  int dims;      // the head's dims
  int scale_f32;
  // Fused bias + RoPE (launch_kv_append_rope only): k/v above are the
  // pre-bias, pre-RoPE rows; q (optional) is rotated into q_out.
  const float* q;  // [n_rows][q_heads*dims], or null
  float* q_out;    // may alias q
  const float* q_bias;  // [q_heads*dims] or null
  const float* k_bias;  // [kv_heads*dims] or null
  const float* v_bias;
  const float* rope_cos;  // [positions][dims/2]
  const float* rope_sin;
  int q_heads;
  int rope_fma;  // 1: one rounding per output (FMA), 0: product, product, sum
};

struct GatherParams {
  const void* pool;  // layer base
  BlockGeom geom;
  const int* table;  // device, the session's page ids
  int count;         // positions to gather
  int kv_heads;
  int head_dim;      // block width
  int dims;          // the head's dims (rows of k_rows / v_rows)
  int scale_bytes;  // 2 or 4
  void* k_rows;
  void* v_rows;
  void* k_scales;  // NULL unless I8
  void* v_scales;
};

struct AttnParams {
  const void* pool;       // layer base: the layer's page blocks
  uint32_t block_bytes;   // block stride
  const SessionRec* sessions;
  const WorkRec* work;
  const int* wg_first;  // [grid+1] first work item of each workgroup, or null
  const int* tables;
  const float* q;  // [rows][q_heads*dims]
  float* out;
  float* part_o;   // [parts][rows_cap][block width]
  float* part_ml;  // [parts][rows_cap][2]: max (log2 domain), sum
  int rows_cap;    // 16 * row groups of the plan
  int kv_heads;
  int q_heads;
  int dims;          // the head's dims
  float scale_log2;  // log2(e) / sqrt(dims)
  // Static sparse subset (sp_stride 0: dense): rows whose span exceeds
  // sp_sink + sp_window keep positions < sp_sink, every sp_stride-th one
  // from sp_sink on, and the last sp_window.
  int sp_sink, sp_window, sp_stride;
  // In-kernel split merge (null: partials are merged by split_reduce_kernel
  // after the launch): the plan's reduction records and one arrival counter
  // each (zero at launch; each record's last piece re-arms it).
  const ReduceRec* reduce;
  int* counters;
  // The step's new K/V rows, [rows][kv_heads*dims] in q's row order, which
  // the launch attends to and stores into the pool (decode variants that
  // can, decode_app_waves; null: the rows are already in the pool). Wave w
  // of workgroup g handles the rows of records [app_first[g*W + w],
  // app_first[g*W + w + 1]) of app_recs: {page id, position, k/v row *
  // kv_heads + KV head, work item} (the plan's build_decode_appends).
  const float* app_k;
  const float* app_v;
  const int* app_first;
  const int* app_recs;
};

struct ReduceParams {
  const ReduceRec* items;
  const float* part_o;
  const float* part_ml;
  float* out;
  int rows_cap;
  int q_heads;
  int dims;  // the head's dims (out's row stride is q_heads * dims)
};

// Small decode step (paged_step_kernel): append + attention + split merge.
struct StepParams {
  AppendParams app;       // pool, geometry, k/v rows, scale format (rows unused)
  const StepRec* recs;    // one per workgroup
  const int* first_ids;   // [workgroups][kStepFirstIds]: the first batch's page ids
  const int* tables;
  const float* q;         // [rows][q_heads*app.dims]
  float* out;
  float* part_o;          // [parts][rows_cap][block width]
  float* part_ml;         // [parts][rows_cap][2]
  int* counters;          // [segments], zero between launches
  int rows_cap;
  int group;              // query heads per KV head
  float scale_log2;
  int sp_sink, sp_window, sp_stride;  // static sparse subset (stride 0: dense)
};

// Kernel-level group attention (tge_attention_group): one KV head's query
// group over positions [first, first + count) of one session's pages.
struct GroupParams {
  const void* pool;      // layer base
  uint32_t block_bytes;  // block stride
  int pages;             // pages of the pool (ids outside give NaN outputs)
  int kv_heads;
  int kv_head;
  const int* page_ids;   // device, the session's block table
  int first;
  int count;
  const float* queries;  // [group_heads][dims]
  int group_heads;
  int dims;              // the head's dims
  float scale;
  float* maxima;         // [group_heads]
  float* sums;           // [group_heads]
  float* accumulators;   // [group_heads][dims]
};

hipError_t launch_kv_append(int format, const AppendParams& p, hipStream_t stream);
// One workgroup per query head of the group.
hipError_t launch_attention_group(int format, int scale_f32, int head_dim, const GroupParams& p,
                                  hipStream_t stream);
// One workgroup per StepRec; row_groups = ceil(max n_new * group / 16).
hipError_t launch_step(int format, int scale_f32, int head_dim, int row_groups, int n_recs,
                       const StepParams& p, hipStream_t stream);
hipError_t launch_kv_append_rope(int format, const AppendParams& p, hipStream_t stream);
hipError_t launch_kv_gather(int format, const GatherParams& p, hipStream_t stream);
// Decode attention over a balanced plan (p.wg_first required): n_groups
// persistent workgroups (a fixed number per CU, see DecodeCfg).
hipError_t launch_decode(int format, int scale_f32, int head_dim, int row_groups, int n_groups,
                         const AttnParams& p, hipStream_t stream);
// Mixed step in one launch (paged_mixed_kernel): n_dec persistent decode
// workgroups over `dec`'s plan (one per CU), then n_pf block-prefill tiles
// of `pf`'s plan; both plans merge their splits in the launch (counters
// required).
hipError_t launch_mixed(int format, int scale_f32, int head_dim, int row_groups, int n_dec,
                        int n_pf, const AttnParams& dec, const AttnParams& pf, hipStream_t stream);
// Block prefill: one workgroup per work item (tiles of up to 128 rows).
// Groups of four waves per block-prefill workgroup (1 or 2): with two, an
// item's pages are shared by both halves and the plan's items may be twice
// as long.
int prefill_halves(int format, int head_dim);
// tile_rows: the plan's tile rows (prefill_tile_rows, or 64 at 128 dims).
hipError_t launch_prefill(int format, int scale_f32, int head_dim, int n_units, int tile_rows,
                          const AttnParams& p, hipStream_t stream);
// Resident decode workgroups per CU (of the static sparse variant when
// `sparse`).
int decode_blocks_per_cu(int format, int scale_f32, int head_dim, int row_groups, bool sparse);
// Waves per workgroup of the dense decode variant if it can store a step's
// new rows (AttnParams::app_k), else 0; decode_app_rows: rows per wave it holds.
int decode_app_waves(int format, int scale_f32, int head_dim, int row_groups);
constexpr int decode_app_rows(int block_dims) { return block_dims <= 64 ? 16 : 8; }
hipError_t launch_reduce(int head_dim, int n_items, int max_parts, const ReduceParams& p,
                         hipStream_t stream);
// Expiries of the kernels' bounded waits since the process started (a
// synchronous read of the device counter).
// Copies n bytes of a pinned host buffer (its device address) to device
// memory on `stream` with a kernel (system-coherent loads).
hipError_t launch_upload(char* dst, const char* src_dev, size_t n, hipStream_t stream);
hipError_t read_wait_expiries(unsigned int* out);
// Read-only streaming of `bytes` (pattern 0: 4 KiB chunks over the grid;
// 1: scattered blocks of block_bytes <= 17 KiB, one wave each).
hipError_t launch_read_ceiling(const void* buf, size_t bytes, int pattern, int workgroups,
                               int block_bytes, hipStream_t stream);

}  // namespace tge
