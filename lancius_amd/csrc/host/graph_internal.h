/*
 * graph_internal.h - symbols shared by the host graph library's sources and
 * not part of its public interface.
 */
#ifndef LANCIUS_AMD_GRAPH_INTERNAL_H
#define LANCIUS_AMD_GRAPH_INTERNAL_H

#include "lancius_graph.h"

/* rt->flags bit (the reference never sets rt->flags): runtime_data was
 * malloc'd by lancius_graph_load and is freed by lancius_graph_destroy. */
#define LANCIUS_RT_FLAG_LOADED 0x100u

/* A zeroed node of `op` with `n_in` input slots, appended to the graph. */
lancius_node* lancius__raw_node(lancius_graph* g, lancius_opcode op, uint8_t ndim, uint32_t n_in);

#endif
