/* TEST INFRASTRUCTURE ONLY (the CPU oracle): internal declarations shared by its files */
#ifndef OSMOS_ORC_INTERNAL_H
#define OSMOS_ORC_INTERNAL_H

#include <stdint.h>

#include "../libosmos_amd/csrc/iq_grids.h"

extern uint64_t orc_grid_iq2xxs[256], orc_grid_iq2xs[512], orc_grid_iq2s[1024], orc_grid_iq1s[2048];
extern uint32_t orc_grid_iq3xxs[256];
extern uint8_t orc_ksigns[128];

static inline uint32_t orc_ld16(const uint8_t *p) { return (uint32_t)p[0] | (uint32_t)p[1] << 8; }
static inline uint32_t orc_ld32(const uint8_t *p) { return orc_ld16(p) | orc_ld16(p + 2) << 16; }
static inline uint64_t orc_ld64(const uint8_t *p) { return (uint64_t)orc_ld32(p) | (uint64_t)orc_ld32(p + 4) << 32; }

#endif
