/* TEST INFRASTRUCTURE ONLY. Built by oracle/Makefile against the reference's own
 * include/glint_cells.h (REF_INCLUDE); writes its GLINT_CELLS table as 1024
 * little-endian f32 bytes to stdout so tests can compare it with ours. */
#include <stdio.h>
#include "glint_cells.h"
int main(void) {
    return fwrite(GLINT_CELLS, sizeof(float), 256, stdout) == 256 ? 0 : 1;
}
