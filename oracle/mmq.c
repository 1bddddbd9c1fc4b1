/* TEST INFRASTRUCTURE ONLY (the CPU oracle; see oracle.h): the mmq contract (Q4_K against int8 activations).

   reference: include/osmos/gpu/mmq.h:7-55 (layouts and contract), kernels/mmq.hip:33-52 (the activations' int8: a
   division, clamped), kernels/mmq.hip:54-151 (the order), tests/gpu/test_mmq_gpu.hip:66-121 (its host replay).
   built with -ffp-contract=off. */
#include <math.h>

#include "oracle.h"
#include "orc_internal.h"

#define GROUP 32
#define SLOTS 16
#define WAVES 4

uint64_t orc_mmq_x8_at(uint32_t s, uint32_t c, uint32_t cols)
{
  return (uint64_t)(s / SLOTS) * SLOTS * cols + (uint64_t)(c / GROUP) * (SLOTS * GROUP) + (s % SLOTS) * GROUP + c % GROUP;
}

uint64_t orc_mmq_dx_at(uint32_t s, uint32_t g, uint32_t groups)
{
  return (uint64_t)(s / SLOTS) * SLOTS * groups + (uint64_t)g * SLOTS + s % SLOTS;
}

bool orc_mmq_x8_rows(const float *x, uint32_t xs, const int32_t *idx, uint32_t slots, uint32_t cols, int8_t *x8,
                     float *dx, float *sx)
{
  if (!x || !idx || !x8 || !dx || !sx || !slots || !cols || cols % GROUP || xs < cols)
    return false;
  const uint32_t groups = cols / GROUP;
  for (uint32_t s = 0; s < slots; s++)
    for (uint32_t g = 0; g < groups; g++)
    {
      float v[GROUP], a = 0.0f;
      for (int i = 0; i < GROUP; i++)
      {
        v[i] = idx[s] >= 0 ? x[(uint64_t)idx[s] * xs + g * GROUP + i] : 0.0f;
        a = fmaxf(a, fabsf(v[i]));
      }
      const float d = a / 127.0f;
      int sum = 0;
      for (int i = 0; i < GROUP; i++)
      {
        const int q = a == 0.0f ? 0 : (int)fminf(fmaxf(rintf(v[i] / d), -127.0f), 127.0f);
        x8[orc_mmq_x8_at(s, g * GROUP + i, cols)] = (int8_t)q;
        sum += q;
      }
      const uint64_t at = orc_mmq_dx_at(s, g, groups);
      dx[at] = a == 0.0f ? 0.0f : d;
      sx[at] = dx[at] * (float)sum;
    }
  return true;
}

/* one row against one slot: partition p its 256-value blocks p, p + 4, ..., each group g in order:
   v = (d sc) dx; acc = fmaf(v, I, acc); acc = fmaf(dmin m, -sx, acc); then the partitions summed in order */
static float mmq_row(const uint8_t *row, uint32_t cols, const int8_t *x8, const float *dx, const float *sx,
                     uint32_t slot)
{
  const uint32_t nb = cols / 256, groups = cols / GROUP;
  float part[WAVES] = {0};
  for (int p = 0; p < WAVES; p++)
    for (uint32_t b = (uint32_t)p; b < nb; b += WAVES)
    {
      const uint8_t *blk = row + (uint64_t)b * 144;
      const float d = orc_f16(orc_ld16(blk)), dmin = orc_f16(orc_ld16(blk + 2));
      const uint8_t *s = blk + 4;
      for (int g = 0; g < 8; g++)
      {
        const int sc = g < 4 ? s[g] & 0x3F : (s[g + 4] & 0x0F) | ((s[g - 4] >> 2) & 0x30);
        const int mn = g < 4 ? s[g + 4] & 0x3F : (s[g + 4] >> 4) | ((s[g] >> 2) & 0x30);
        const float dsc = d * (float)sc, dm = dmin * (float)mn;
        const uint32_t gg = b * 8 + (uint32_t)g;
        int isum = 0;
        for (int i = 0; i < GROUP; i++)
          isum += ((blk[16 + (g / 2) * 32 + i] >> (4 * (g % 2))) & 0x0F) * x8[orc_mmq_x8_at(slot, gg * GROUP + i, cols)];
        const uint64_t at = orc_mmq_dx_at(slot, gg, groups);
        const float v = dsc * dx[at];
        part[p] = fmaf(v, (float)isum, part[p]);
        part[p] = fmaf(dm, -sx[at], part[p]);
      }
    }
  float r = part[0];
  for (int p = 1; p < WAVES; p++)
    r = r + part[p];
  return r;
}

bool orc_mmq_rows(const void *w, uint32_t cols, uint32_t r0, uint32_t r1, const int8_t *x8, const float *dx,
                  const float *sx, uint32_t slot, float *y)
{
  if (!w || !x8 || !dx || !sx || !y || !cols || cols % 256 || r1 < r0)
    return false;
  const uint64_t rb = (uint64_t)(cols / 256) * 144;
  for (uint32_t r = r0; r < r1; r++)
    y[r] = mmq_row((const uint8_t *)w + r * rb, cols, x8, dx, sx, slot);
  return true;
}
