/* libosmos MI355X: the lane's CPU half (drop-in for the reference's include/osmos/cpu/lane.h:1-44, src/cpu/lane.c) - a
   layer's experts that are not in GPU memory computed by a pool of host threads, the bits the GPU's lane gives them
   (q8_round, q8_gate_up, q8_round, q8_group_tok: the lane contract, reference kernels/lane.h:43-75, kernels/q8.h), for
   the GPU to take once the job's flag is posted (ops_wait, then ops_copy_rows: reference src/run/hip_lane.c:205-222).
   contracts: reference include/osmos/cpu/lane.h:46-74. */
#ifndef CPU_LANE_H
#define CPU_LANE_H

#include <stdbool.h>
#include <stdint.h>

#define CPU_LANE_THREADS_MAX 64       /* reference include/osmos/cpu/lane.h:7: a pool's most workers */
#define CPU_LANE_FAILED 0x80000000u   /* reference include/osmos/cpu/lane.h:8: a failed job's posted value carries it */

#ifdef __cplusplus
extern "C" {
#endif

typedef struct CpuLane CpuLane;

/* reference include/osmos/cpu/lane.h:12-19: an expert of a job - its three matrices in host memory (gate and up ff
   rows of dim, down dim rows of ff) and its rows of the job's x, row0 .. row0 + cnt */
typedef struct CpuLaneExpert
{
  const void *gate, *up, *down;
  uint32_t row0, cnt;
} CpuLaneExpert;

/* reference include/osmos/cpu/lane.h:21-34 */
typedef struct CpuLaneJob
{
  uint32_t type_gu, type_down; /* the experts' types: the lane's (q8.h) */
  uint32_t dim, ff;
  float lim;                   /* the activation's clamp */
  const float *x;              /* n_rows rows of dim: row r a (token, expert) pair's input */
  const float *scale;          /* row r's routed weight */
  uint32_t n_rows;
  const CpuLaneExpert *e;
  uint32_t n_e;
  float *y;                    /* row r's output at y + r dim */
  uint32_t *seq;               /* where `value` is posted when the job is done (release), | CPU_LANE_FAILED if not */
  uint32_t value;
} CpuLaneJob;

/* replaces reference include/osmos/cpu/lane.h:36 (src/cpu/lane.c:158-207): `threads` workers (1 ..
   CPU_LANE_THREADS_MAX), jobs of at most max_rows rows of dim and ff (multiples of 256); cores NULL (the scheduler
   places them) or `threads` logical CPUs, worker i pinned to cores[i] from its start (NULL where one cannot be). NULL
   for a size it cannot take, or a thread or memory refused. (the reference also refuses a CPU without its AVX-512
   kernels; this one runs on any x86-64 or other host) */
CpuLane *cpu_lane_create(int threads, const int *cores, uint32_t max_rows, uint32_t dim, uint32_t ff);
/* replaces reference include/osmos/cpu/lane.h:37: waits for a job under way, joins the workers, frees; NULL: nothing */
void cpu_lane_destroy(CpuLane *c);
/* replaces reference include/osmos/cpu/lane.h:38 (src/cpu/lane.c:231-245): queues one job and returns at once - x's
   rows rounded, each expert's gate and up rows with the activation, the activations rounded, the down rows, the
   rows of each phase split over the workers; the last worker posts seq. false, nothing queued and seq untouched, for
   a job under way, a type that is not the lane's, dim or ff not the pool's, rows past max_rows or an expert's past
   n_rows, or no outputs */
bool cpu_lane_submit(CpuLane *c, const CpuLaneJob *job);
/* replaces reference include/osmos/cpu/lane.h:39: waits for the job under way; true if it and every job since the
   last wait succeeded */
bool cpu_lane_wait(CpuLane *c);

#ifdef __cplusplus
}
#endif

#endif
