/* Umbrella header of the CLSamp system-library module: the C ABI of the
 * MI355X sampling stage (liblsamp.so).  The module map sits beside this file,
 * as the reference's xgrammar module map sits beside xgrammar_c.h
 * (Libraries/MLXCXGrammar/include/module.modulemap). */
#include "../../../include/lsamp.h"
