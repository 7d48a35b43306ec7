// repack.h — host-side conversion into the resident device layout (fmt.h).
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <vector>

#include "mynah_asr_hip.h"

struct HostLayout {
    std::vector<uint8_t> p0, p1, h;
    std::vector<float> h2;
    int Np = 0, Kp = 0;
};

// Block geometry of a format (elements, bytes). -1 for an unknown format.
int mh_format_info(int qtype, int *block_elems, int *block_bytes);
// 0 on success; -1 for an unsupported format or shape.
int mh_repack(const mynah_asr_hip_wdesc *w, HostLayout *L);
// Total device bytes and the 256-aligned offsets of p0, p1, h, h2.
size_t mh_layout_bytes(const HostLayout &L, size_t off[4]);
