"""Pool layout and block bookkeeping the decode runner needs."""
