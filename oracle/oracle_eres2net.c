/* oracle_eres2net.c - placeholder until the ERes2Net restatement lands. TEST INFRASTRUCTURE ONLY. */
