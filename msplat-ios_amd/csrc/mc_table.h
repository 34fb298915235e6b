// mc_table.h -- the marching-cubes case table, generated at compile time.
//
// Cube corners and edges are numbered as the reference numbers them
// (core/metal/msplat_metal.metal:2594-2604): corner c sits at kCorner[c]
// (x, y, z offsets), edge e joins corners kEdge[e].  A case is the 8-bit
// mask of corners whose SDF is negative ("inside", :2635-2638).
//
// The triangles of a case are derived, not tabulated by hand:
//   1. On each face of the cube, every maximal run of inside corners (walking
//      the face's corners counter-clockwise as seen from outside) is cut off
//      by one segment between the crossings on the two edges that leave the
//      run.  A face whose two inside corners sit on a diagonal therefore gets
//      two segments (the inside corners stay separated); a neighbouring cell
//      sees the same face with the same corner signs and makes the same
//      segments, so the surfaces of adjacent cells meet edge to edge.
//   2. The segments of all six faces chain into closed loops (every crossed
//      edge ends one segment and starts another).
//   3. Each loop (3 to 7 crossings) is triangulated as a fan from its first
//      crossing whose fan diagonals join crossings on no common face, so no
//      triangle edge other than the face segments lies in a face plane
//      (such an edge could coincide with the neighbouring cell's).
// Triangles are wound so that their right-hand normal points towards the
// inside (negative-SDF) corners, the winding of the reference's table (its
// case 1, corner 0 inside, is the triangle of edges 0, 8, 3 whose normal
// points at corner 0).  At most 5 triangles per case.
#pragma once

#include <stdint.h>

namespace mcgen {

constexpr int kCorner[8][3] = {{0, 0, 0}, {1, 0, 0}, {1, 1, 0}, {0, 1, 0},
                               {0, 0, 1}, {1, 0, 1}, {1, 1, 1}, {0, 1, 1}};
constexpr int kEdge[12][2] = {{0, 1}, {1, 2}, {2, 3}, {3, 0}, {4, 5}, {5, 6},
                              {6, 7}, {7, 4}, {0, 4}, {1, 5}, {2, 6}, {3, 7}};
// Faces as corner cycles, counter-clockwise seen from outside the cube
// (x = 0, x = 1, y = 0, y = 1, z = 0, z = 1), and the edge that joins
// kFace[f][i] to kFace[f][(i + 1) % 4].
constexpr int kFace[6][4] = {{4, 7, 3, 0}, {1, 2, 6, 5}, {0, 1, 5, 4},
                             {7, 6, 2, 3}, {3, 2, 1, 0}, {4, 5, 6, 7}};
constexpr int kFaceEdge[6][4] = {{7, 11, 3, 8}, {1, 10, 5, 9}, {0, 9, 4, 8},
                                 {6, 10, 2, 11}, {2, 1, 0, 3}, {4, 5, 6, 7}};

struct McTable {
    int8_t tri[256][16];  // edge indices, 3 per triangle, -1 terminated
    uint8_t ntri[256];    // triangles per case
    uint16_t edges[256];  // bit e set: edge e is crossed
};

constexpr int face_mask(int e) {
    int m = 0;
    for (int f = 0; f < 6; ++f)
        for (int i = 0; i < 4; ++i)
            if (kFaceEdge[f][i] == e) m |= 1 << f;
    return m;
}

constexpr McTable make_mc_table() {
    McTable t{};
    int fm[12] = {};
    for (int e = 0; e < 12; ++e) fm[e] = face_mask(e);
    for (int m = 0; m < 256; ++m) {
        for (int i = 0; i < 16; ++i) t.tri[m][i] = -1;
        int next[12] = {};
        int first[12] = {};
        int nseg = 0;
        for (int f = 0; f < 6; ++f) {
            bool in[4] = {};
            int cnt = 0;
            for (int i = 0; i < 4; ++i) {
                in[i] = ((m >> kFace[f][i]) & 1) != 0;
                cnt += in[i] ? 1 : 0;
            }
            if (cnt == 0 || cnt == 4) continue;
            for (int k = 0; k < 4; ++k) {
                if (!in[k] || in[(k + 3) % 4]) continue;  // k starts a run
                int j = k;
                while (in[(j + 1) % 4]) j = (j + 1) % 4;
                const int enter = kFaceEdge[f][(k + 3) % 4];  // crossing before the run
                const int leave = kFaceEdge[f][j];            // crossing after the run
                next[leave] = enter;  // inward winding
                first[nseg++] = leave;
            }
        }
        bool used[12] = {};
        int nt = 0;
        uint16_t crossed = 0;
        for (int s = 0; s < nseg; ++s) {
            const int a = first[s];
            if (used[a]) continue;
            int loop[12] = {};
            int n = 0;
            int cur = a;
            do {
                loop[n++] = cur;
                used[cur] = true;
                crossed = (uint16_t)(crossed | (1u << cur));
                cur = next[cur];
            } while (cur != a);
            int s0 = 0;
            for (int st = 0; st < n; ++st) {
                bool clean = true;
                for (int d = 2; d < n - 1; ++d)
                    if (fm[loop[st]] & fm[loop[(st + d) % n]]) clean = false;
                if (clean) {
                    s0 = st;
                    break;
                }
            }
            for (int d = 1; d < n - 1; ++d) {
                t.tri[m][3 * nt + 0] = (int8_t)loop[s0];
                t.tri[m][3 * nt + 1] = (int8_t)loop[(s0 + d) % n];
                t.tri[m][3 * nt + 2] = (int8_t)loop[(s0 + d + 1) % n];
                ++nt;
            }
        }
        t.ntri[m] = (uint8_t)nt;
        t.edges[m] = crossed;
    }
    return t;
}

}  // namespace mcgen
