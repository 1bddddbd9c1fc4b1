/* TEST INFRASTRUCTURE ONLY (the CPU oracle; see oracle.h): shared pieces - f16 decoding, the block table and the
   codebooks expanded from libosmos_amd/csrc/iq_grids.h's packed indices. */
#include <string.h>

#include "oracle.h"
#include "orc_internal.h"

uint64_t orc_grid_iq2xxs[256], orc_grid_iq2xs[512], orc_grid_iq2s[1024], orc_grid_iq1s[2048];
uint32_t orc_grid_iq3xxs[256];
uint8_t orc_ksigns[128];
static int ready;

void orc_init(void)
{
  if (ready)
    return;
  for (int i = 0; i < 256; i++)
    orc_grid_iq2xxs[i] = iq_expand8(iq_packed_iq2xxs[i], iq_map_iq2);
  for (int i = 0; i < 512; i++)
    orc_grid_iq2xs[i] = iq_expand8(iq_packed_iq2xs[i], iq_map_iq2);
  for (int i = 0; i < 1024; i++)
    orc_grid_iq2s[i] = iq_expand8(iq_packed_iq2s[i], iq_map_iq2);
  for (int i = 0; i < 2048; i++)
    orc_grid_iq1s[i] = iq_expand8(iq_packed_iq1s[i], iq_map_iq1);
  for (int i = 0; i < 256; i++)
    orc_grid_iq3xxs[i] = iq_expand4(iq_packed_iq3xxs[i]);
  for (int i = 0; i < 128; i++)
    orc_ksigns[i] = iq_ksign((uint32_t)i);
  ready = 1;
}

/* the expanded tables as bytes, for the tests' checksums against the reference's */
const void *orc_table(int which, uint32_t *bytes)
{
  orc_init();
  switch (which)
  {
  case 0: *bytes = sizeof orc_grid_iq2xxs; return orc_grid_iq2xxs;
  case 1: *bytes = sizeof orc_grid_iq2xs; return orc_grid_iq2xs;
  case 2: *bytes = sizeof orc_grid_iq2s; return orc_grid_iq2s;
  case 3: *bytes = sizeof orc_grid_iq1s; return orc_grid_iq1s;
  case 4: *bytes = sizeof orc_grid_iq3xxs; return orc_grid_iq3xxs;
  case 5: *bytes = sizeof orc_ksigns; return orc_ksigns;
  default: *bytes = 0; return 0;
  }
}

/* IEEE half to float, exact (subnormals and infinities included) */
float orc_f16(uint32_t bits)
{
  const uint32_t s = (bits >> 15) & 1, e = (bits >> 10) & 0x1F, m = bits & 0x3FF;
  uint32_t f;
  if (e == 0)
  {
    if (m == 0)
      f = s << 31;
    else
    { /* subnormal: m * 2^-24, normalised */
      int sh = 0;
      uint32_t mm = m;
      while (!(mm & 0x400))
        mm <<= 1, sh++;
      f = (s << 31) | ((uint32_t)(113 - sh) << 23) | ((mm & 0x3FF) << 13);
    }
  }
  else if (e == 31)
    f = (s << 31) | 0x7F800000u | (m << 13);
  else
    f = (s << 31) | ((e + 112) << 23) | (m << 13);
  float r;
  memcpy(&r, &f, sizeof r);
  return r;
}

/* reference include/osmos/model/qtype.h:28-53 (values, bytes) */
uint32_t orc_block_values(uint32_t type)
{
  switch (type)
  {
  case ORC_F32:
  case ORC_BF16: return 1;
  case ORC_Q4_0:
  case ORC_Q8_0:
  case ORC_IQ4_NL: return 32;
  case ORC_Q2_K:
  case ORC_Q3_K:
  case ORC_Q4_K:
  case ORC_Q5_K:
  case ORC_Q6_K:
  case ORC_IQ2_XXS:
  case ORC_IQ2_XS:
  case ORC_IQ3_XXS:
  case ORC_IQ1_S:
  case ORC_IQ2_S:
  case ORC_IQ4_XS:
  case ORC_IQ1_M: return 256;
  default: return 0;
  }
}

uint32_t orc_block_bytes(uint32_t type)
{
  switch (type)
  {
  case ORC_F32: return 4;
  case ORC_BF16: return 2;
  case ORC_Q4_0: return 18;
  case ORC_Q8_0: return 34;
  case ORC_IQ4_NL: return 18;
  case ORC_Q2_K: return 84;
  case ORC_Q3_K: return 110;
  case ORC_Q4_K: return 144;
  case ORC_Q5_K: return 176;
  case ORC_Q6_K: return 210;
  case ORC_IQ2_XXS: return 66;
  case ORC_IQ2_XS: return 74;
  case ORC_IQ3_XXS: return 98;
  case ORC_IQ1_S: return 50;
  case ORC_IQ2_S: return 82;
  case ORC_IQ4_XS: return 136;
  case ORC_IQ1_M: return 56;
  default: return 0;
  }
}
